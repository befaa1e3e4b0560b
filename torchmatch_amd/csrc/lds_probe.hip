// lds_probe.hip -- LDS read-bandwidth microbenchmark for gfx950.
//
// Measurement support only (not part of the C ABI in include/): the JV
// kernels keep their cost tiles in LDS, and their roofline is priced against
// the chip's LDS read bandwidth.  This kernel measures that peak on the box:
// every workgroup fills 16 KiB of LDS once, then each lane streams 16-byte
// reads (ds_read_b128, consecutive lanes on consecutive 16-byte words, so no
// bank conflicts) and folds them with XOR so the loads cannot be dropped.
// Eight 256-lane workgroups fit per CU (128 KiB of the 160 KiB LDS).
#include <hip/hip_runtime.h>
#include <stdint.h>

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

} // namespace

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
