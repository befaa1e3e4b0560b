// jv_unpack.hip -- device unpack of a packed row->col mapping (gfx950).
//
// Produces the tuple of torchmatch's `assignment::jonker_dense_batch_unpacked`
// (sources/torchmatch/assignment/cpu/ops.cpp:291-417, the unpack loop at
// :387-414) from the (B, N) int64 mapping the solver writes:
//   matches         (B, N, 2)  (row, col) of the matched rows in row order,
//                              -1 past n_matches[b]
//   unmatched_rows  (B, N)     unmatched rows in increasing order, -1 after
//   unmatched_cols  (B, M)     columns no row took, increasing, -1 after
//   n_matches       (B,)
// One 64-lane workgroup per problem.  Each 64-row (or 64-column) chunk is
// compacted with a ballot and a per-lane popcount of the lanes below, so the
// order is the sequential loop's; used columns are marked in an LDS bitmap.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "jv_batch.h"
#include "wave.h"

namespace tmamd {
namespace {

constexpr int kUnpackMaxM = 4096;  // columns the LDS bitmap covers

__global__ void __launch_bounds__(64)
jv_unpack_kernel(const int64_t *__restrict__ packed, int N, int M,
                 int64_t *__restrict__ matches, int64_t *__restrict__ unmatched_rows,
                 int64_t *__restrict__ unmatched_cols, int64_t *__restrict__ n_matches) {
    __shared__ uint32_t used[kUnpackMaxM / 32];
    const int lane = lane_id();
    const int64_t b = blockIdx.x;
    const int64_t *pk = packed + b * N;
    int64_t *mb = matches + b * (int64_t)N * 2;
    int64_t *urb = unmatched_rows + b * N;
    int64_t *ucb = unmatched_cols + b * M;
    for (int w = lane; w < (M + 31) / 32; w += 64)
        used[w] = 0;
    __syncthreads();
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    int nm = 0, nur = 0;
    for (int base = 0; base < N; base += 64) {
        const int i = base + lane;
        const int64_t j = i < N ? pk[i] : -1;
        const bool hit = i < N && j >= 0 && j < M;
        const uint64_t hm = ballot(hit);
        const uint64_t um = ballot(i < N && !hit);
        if (hit) {
            const int slot = nm + __builtin_popcountll(hm & below);
            mb[2 * slot] = i;
            mb[2 * slot + 1] = j;
            atomicOr(&used[j >> 5], 1u << (j & 31));
        } else if (i < N) {
            urb[nur + __builtin_popcountll(um & below)] = i;
        }
        nm += __builtin_popcountll(hm);
        nur += __builtin_popcountll(um);
    }
    __syncthreads();
    int nuc = 0;
    for (int base = 0; base < M; base += 64) {
        const int j = base + lane;
        const bool free_col = j < M && ((used[j >> 5] >> (j & 31)) & 1u) == 0;
        const uint64_t fm = ballot(free_col);
        if (free_col)
            ucb[nuc + __builtin_popcountll(fm & below)] = j;
        nuc += __builtin_popcountll(fm);
    }
    // -1 padding past the valid prefixes, as the CPU op's at::full(-1) leaves
    for (int k = nm * 2 + lane; k < 2 * N; k += 64)
        mb[k] = -1;
    for (int k = nur + lane; k < N; k += 64)
        urb[k] = -1;
    for (int k = nuc + lane; k < M; k += 64)
        ucb[k] = -1;
    if (lane == 0)
        n_matches[b] = nm;
}

} // namespace
} // namespace tmamd

extern "C" int tm_jv_unpack_i64(const int64_t *packed, int64_t B, int32_t N, int32_t M,
                                int64_t *matches, int64_t *unmatched_rows,
                                int64_t *unmatched_cols, int64_t *n_matches,
                                hipStream_t stream) {
    if (B < 0 || N < 0 || M < 0)
        return TM_ERR_INVALID_ARGUMENT;
    if (B == 0)
        return TM_OK;
    if (packed == nullptr || matches == nullptr || unmatched_rows == nullptr ||
        unmatched_cols == nullptr || n_matches == nullptr)
        return TM_ERR_INVALID_ARGUMENT;
    if (M > tmamd::kUnpackMaxM || B > (int64_t)0x7fffffff)
        return TM_ERR_UNSUPPORTED_SHAPE;
    hipLaunchKernelGGL(tmamd::jv_unpack_kernel, dim3((unsigned)B), dim3(64), 0, stream, packed,
                       (int)N, (int)M, matches, unmatched_rows, unmatched_cols, n_matches);
    return hipGetLastError() == hipSuccess ? TM_OK : TM_ERR_LAUNCH;
}
