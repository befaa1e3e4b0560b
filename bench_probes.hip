// bench_probes.hip -- gfx950 microbenchmarks bench.py prices the JV kernels
// against (measurement support for the benchmark, not part of the library).
//
// 1. LDS read bandwidth: the north star prices JV against the chip's LDS
//    read bandwidth.  Every workgroup fills 16 KiB of LDS once, then each lane
//    streams 16-byte reads (ds_read_b128, consecutive lanes on consecutive
//    16-byte words, so no bank conflicts) and folds them with XOR so the loads
//    cannot be dropped.  Eight 256-lane workgroups fit per CU (128 KiB of the
//    160 KiB LDS).
// 2. Wave-wide argmin latency: one step of the JV kernel's shortest-path
//    search needs the minimum key over the 64 columns (wave_min_key_s of
//    torchmatch_amd/csrc/wave.h) and the lane holding it before the next step
//    can start, so a chain of them is the floor of a search.  One wave runs
//    `iters` dependent (minimum, argmin lane) rounds and records core-clock
//    cycles (s_memtime) and wall time (s_memrealtime, 100 MHz), which also
//    gives the shader clock.
// 3. Streaming HBM read: what one kernel that reads a buffer once reaches on
//    this chip, the practical ceiling of the Sinkhorn pass.  Each workgroup
//    reads its own contiguous range with eight 16-byte non-temporal loads per
//    lane in flight (the fastest layout of a sweep over grid-stride and
//    contiguous ranges, ordinary and non-temporal loads) and folds them so
//    the loads cannot be dropped.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "torchmatch_amd/csrc/wave.h"

namespace {

constexpr int kProbeThreads = 256;
constexpr int kProbeWords = 1024;  // uint4 words = 16 KiB per workgroup

__global__ void __launch_bounds__(kProbeThreads)
lds_read_probe(uint32_t *__restrict__ sink, int iters) {
    __shared__ uint4 buf[kProbeWords];
    const int t = threadIdx.x;
    for (int k = t; k < kProbeWords; k += kProbeThreads)
        buf[k] = make_uint4(k, k * 3u, k * 5u, k * 7u);
    __syncthreads();
    uint4 acc = make_uint4(0, 0, 0, 0);
#pragma unroll 8
    for (int i = 0; i < iters; ++i) {
        const uint4 a = buf[(t + i * 64) & (kProbeWords - 1)];
        acc.x ^= a.x;
        acc.y ^= a.y;
        acc.z ^= a.z;
        acc.w ^= a.w;
    }
    const uint32_t r = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (r == 0x9e3779b9u)  // practically never: keeps the loop alive
        sink[blockIdx.x] = r;
}

__global__ void __launch_bounds__(64)
argmin_chain_probe(const float *__restrict__ in, unsigned long long *__restrict__ out,
                   int iters) {
    using namespace tmamd;
    const int lane = lane_id();
    int key = __float_as_int(in[lane]);
    const unsigned long long c0 = __builtin_amdgcn_s_memtime();
    const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
        const int kmin = wave_min_key_s(key);
        const int js = first_lane(ballot(key == kmin));
        key = lane == js ? key + 1 : key;
    }
    const unsigned long long c1 = __builtin_amdgcn_s_memtime();
    const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    if (lane == 0) {
        out[0] = c1 - c0;
        out[1] = r1 - r0;
        out[2] = (unsigned long long)(unsigned)key;
    }
}

typedef float vf4 __attribute__((ext_vector_type(4)));
constexpr int kReadUnroll = 8;

__global__ void __launch_bounds__(kProbeThreads)
hbm_read_probe(const vf4 *__restrict__ src, size_t n4, size_t per_block,
               float *__restrict__ sink) {
    const size_t begin = (size_t)blockIdx.x * per_block;
    const size_t end = begin + per_block < n4 ? begin + per_block : n4;
    vf4 acc = {0.f, 0.f, 0.f, 0.f};
    for (size_t i = begin + threadIdx.x; i < end; i += kReadUnroll * kProbeThreads) {
        vf4 v[kReadUnroll];
#pragma unroll
        for (int u = 0; u < kReadUnroll; ++u) {
            const size_t k = i + (size_t)u * kProbeThreads;
            v[u] = __builtin_nontemporal_load(src + (k < end ? k : end - 1));
        }
#pragma unroll
        for (int u = 0; u < kReadUnroll; ++u)
            if (i + (size_t)u * kProbeThreads < end)
                acc += v[u];
    }
    const float s = acc.x + acc.y + acc.z + acc.w;
    if (s == -1234.5f)  // keeps the loads; sink has a word per workgroup
        sink[blockIdx.x] = s;
}

} // namespace

// One wave runs `iters` dependent argmin rounds over 64 floats `in` (device,
// 64 floats); out[0] = core cycles, out[1] = 100 MHz ticks (3 words of
// device memory).  Synchronises the stream; returns 0, or -1 on an error.
extern "C" int tm_probe_argmin_chain(const float *in, unsigned long long *out, int iters,
                                     hipStream_t stream) {
    if (in == nullptr || out == nullptr || iters <= 0)
        return -1;
    hipLaunchKernelGGL(argmin_chain_probe, dim3(1), dim3(64), 0, stream, in, out, iters);
    if (hipGetLastError() != hipSuccess)
        return -1;
    return hipStreamSynchronize(stream) == hipSuccess ? 0 : -1;
}

// Runs the probe once on `stream` with `blocks` workgroups of 256 lanes, each
// lane issuing `iters` 16-byte LDS reads; returns the bytes read (0 on a
// launch error).  `sink` needs `blocks` words of device memory.
extern "C" int64_t tm_probe_lds_read(uint32_t *sink, int blocks, int iters,
                                     hipStream_t stream) {
    if (blocks <= 0 || iters <= 0 || sink == nullptr)
        return 0;
    hipLaunchKernelGGL(lds_read_probe, dim3((unsigned)blocks), dim3(kProbeThreads), 0, stream,
                       sink, iters);
    if (hipGetLastError() != hipSuccess)
        return 0;
    return (int64_t)blocks * kProbeThreads * (int64_t)iters * 16;
}

// Reads `bytes` (a multiple of 16, > 0) of device memory at `src` once, split
// into `blocks` contiguous ranges of 256-lane workgroups, on `stream`;
// returns the bytes read (0 on a bad argument or a launch error).  `sink`
// needs `blocks` floats of device memory.
extern "C" int64_t tm_probe_hbm_read(const void *src, size_t bytes, float *sink, int blocks,
                                     hipStream_t stream) {
    if (src == nullptr || sink == nullptr || blocks <= 0 || bytes < 16 || bytes % 16 != 0)
        return 0;
    const size_t n4 = bytes / 16;
    const size_t per_block = (n4 + (size_t)blocks - 1) / (size_t)blocks;
    hipLaunchKernelGGL(hbm_read_probe, dim3((unsigned)blocks), dim3(kProbeThreads), 0, stream,
                       static_cast<const vf4 *>(src), n4, per_block, sink);
    if (hipGetLastError() != hipSuccess)
        return 0;
    return (int64_t)bytes;
}
