// sinkhorn.hip -- log-domain Sinkhorn (balanced and unbalanced) for gfx950.
//
// Computes what torchmatch's pure-PyTorch reference computes:
//   transport/matrix/_log_sinkhorn.py:136-221     (log_sinkhorn_plan)
//   transport/matrix/_unbalanced_sinkhorn.py:30-103 (unbalanced_sinkhorn_plan)
// per step with epsilon e (schedule from transport/matrix/_schedule.py:21-76):
//   K        = -C / e                                 (float32 IEEE division)
//   lse_c[i] = LSE_j(K[i,j] + log_v[j]),  -inf for rows of C that are all +inf
//   log_u[i] = isfinite(lse_c) ? damp*(log_mu[i] - lse_c[i]) : log_u[i]
//   lse_r[j] = LSE_i(K[i,j] + log_u[i]),  -inf for columns that are all +inf
//   log_v[j] = isfinite(lse_r) ? damp*(log_nu[j] - lse_r[j]) : log_v[j]
// (damp = 1 balanced, 1/(1 + e/rho) unbalanced; torch.logsumexp's shift rule:
// the max, replaced by 0 when it is +-inf) and finally
//   log_plan = (log_u[i] + (-C/e_final)) + log_v[j].
// The reference's -80 stand-in for all-+inf rows/columns only feeds lanes that
// the reference then overwrites with -inf, so those sweeps are skipped here.
//
// Data layout (all row-major, float32, resident in HBM for the whole call):
//   K       (B, N, M)  log kernel, rewritten only when the schedule's epsilon
//                      changes (once for a constant schedule)
//   log_u/v (B, N) / (B, M) caller's outputs, updated in place every step
//   colpart (B, n_chunk, M) float2 (max, sum) column partials
// Per step: row sweep (reads K once), column sweep (reads K once), merge.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "jv_batch.h"
#include "wave.h"

namespace tmamd {
namespace {

constexpr int kRowBlock = 256;            // 4 waves, one row per wave
constexpr int kColBlock = 256;            // 4 columns per thread
constexpr int kColStrip = kColBlock * 4;  // columns per column-sweep block
constexpr int kMapBlock = 256;

__device__ __forceinline__ float f_inf() { return __int_as_float(0x7f800000); }

struct SinkhornLayout {
    int64_t B, N, M;
    int n_chunk;      // row chunks of the column sweep
    int rows_per_chunk;
    int n_strip;      // column strips of the column sweep
    size_t off_k, off_logmu, off_lognu, off_infrow, off_infcol, off_colpart, total;
};

__host__ __device__ inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

SinkhornLayout make_layout(int64_t B, int64_t N, int64_t M) {
    SinkhornLayout L{};
    L.B = B;
    L.N = N;
    L.M = M;
    L.n_strip = (int)((M + kColStrip - 1) / kColStrip);
    // aim for ~2048 column-sweep blocks, at least 16 rows per chunk
    int64_t want = 2048 / (B * L.n_strip > 0 ? B * L.n_strip : 1);
    if (want < 1)
        want = 1;
    int64_t rpc = (N + want - 1) / want;
    if (rpc < 16)
        rpc = 16;
    L.rows_per_chunk = (int)rpc;
    L.n_chunk = (int)((N + rpc - 1) / rpc);
    size_t off = 0;
    L.off_k = off;
    off = align_up(off + sizeof(float) * (size_t)(B * N * M), 256);
    L.off_logmu = off;
    off = align_up(off + sizeof(float) * (size_t)(B * N), 256);
    L.off_lognu = off;
    off = align_up(off + sizeof(float) * (size_t)(B * M), 256);
    L.off_infrow = off;
    off = align_up(off + (size_t)(B * N), 256);
    L.off_infcol = off;
    off = align_up(off + (size_t)(B * M), 256);
    L.off_colpart = off;
    off = align_up(off + sizeof(float2) * (size_t)B * L.n_chunk * (size_t)M, 256);
    L.total = off;
    return L;
}

// ---- elementwise preparation ------------------------------------------------

// K = -C / e (IEEE division, as torch's `-cost / step_eps` in float32).
__global__ void __launch_bounds__(kMapBlock)
sk_log_kernel(const float *__restrict__ C, float *__restrict__ K, int64_t n, float eps) {
    const int64_t stride = (int64_t)gridDim.x * kMapBlock;
    const int64_t n4 = n / 4;
    const float4 *c4 = reinterpret_cast<const float4 *>(C);
    float4 *k4 = reinterpret_cast<float4 *>(K);
    for (int64_t k = (int64_t)blockIdx.x * kMapBlock + threadIdx.x; k < n4; k += stride) {
        const float4 c = c4[k];
        float4 r;
        r.x = -c.x / eps;
        r.y = -c.y / eps;
        r.z = -c.z / eps;
        r.w = -c.w / eps;
        k4[k] = r;
    }
    for (int64_t k = n4 * 4 + (int64_t)blockIdx.x * kMapBlock + threadIdx.x; k < n; k += stride)
        K[k] = -C[k] / eps;
}

// log of the marginals (torch `a.log()`), n elements.
__global__ void __launch_bounds__(kMapBlock)
sk_log_marginal(const float *__restrict__ x, float *__restrict__ y, int64_t n) {
    const int64_t k = (int64_t)blockIdx.x * kMapBlock + threadIdx.x;
    if (k < n)
        y[k] = logf(x[k]);
}

__global__ void __launch_bounds__(kMapBlock)
sk_fill(float *__restrict__ y, int64_t n, float value) {
    const int64_t k = (int64_t)blockIdx.x * kMapBlock + threadIdx.x;
    if (k < n)
        y[k] = value;
}

// inf_row[b, i] = all_j C[b, i, j] == +inf (one wave per row).
__global__ void __launch_bounds__(kRowBlock)
sk_inf_rows(const float *__restrict__ C, uint8_t *__restrict__ inf_row, int64_t rows,
            int64_t M) {
    const int64_t r = (int64_t)blockIdx.x * (kRowBlock / 64) + threadIdx.x / 64;
    if (r >= rows)
        return;
    const float *row = C + r * M;
    bool all_inf = true;
    for (int64_t j = lane_id(); j < M; j += 64)
        all_inf = all_inf && (row[j] == f_inf());
    const bool any_finite = ballot(!all_inf) != 0;
    if (lane_id() == 0)
        inf_row[r] = any_finite ? 0 : 1;
}

// inf_col[b, j] = all_i C[b, i, j] == +inf (one thread per column; runs once).
__global__ void __launch_bounds__(kMapBlock)
sk_inf_cols(const float *__restrict__ C, uint8_t *__restrict__ inf_col, int64_t B, int64_t N,
            int64_t M) {
    const int64_t t = (int64_t)blockIdx.x * kMapBlock + threadIdx.x;
    if (t >= B * M)
        return;
    const int64_t b = t / M, j = t % M;
    const float *col = C + b * N * M + j;
    bool all_inf = true;
    for (int64_t i = 0; i < N && all_inf; ++i)
        all_inf = col[i * M] == f_inf();
    inf_col[t] = all_inf ? 1 : 0;
}

// ---- log-sum-exp helpers --------------------------------------------------------

// Running (shift, sum) pair: sum = sum_k exp(t_k - shift), where shift is the
// running max, or 0 while that max is -inf (torch.logsumexp's rule).
struct Lse {
    float m;  // running max (may be -inf)
    float s;  // sum of exp(t - shift(m))
};

__device__ __forceinline__ float lse_shift(float m) { return isinf(m) ? 0.f : m; }

// Combine two partial pairs.
__device__ __forceinline__ Lse lse_merge(Lse p, Lse q) {
    const float m = fmaxf(p.m, q.m);
    const float sh = lse_shift(m);
    const float a = (p.s == 0.f) ? 0.f : p.s * expf(lse_shift(p.m) - sh);
    const float c = (q.s == 0.f) ? 0.f : q.s * expf(lse_shift(q.m) - sh);
    return Lse{m, a + c};
}

__device__ __forceinline__ float lse_value(Lse p) {
    return logf(p.s) + lse_shift(p.m);
}

// Fold a group of values t[0..G) into a running pair (rescale once per group).
template <int G>
__device__ __forceinline__ void lse_push(Lse &acc, const float (&t)[G]) {
    float gm = t[0];
#pragma unroll
    for (int k = 1; k < G; ++k)
        gm = fmaxf(gm, t[k]);
    if (gm > acc.m) {
        if (acc.s != 0.f)
            acc.s *= expf(lse_shift(acc.m) - lse_shift(gm));
        acc.m = gm;
    }
    const float sh = lse_shift(acc.m);
    float add = 0.f;
#pragma unroll
    for (int k = 0; k < G; ++k)
        add += expf(t[k] - sh);
    acc.s += add;
}

__device__ __forceinline__ Lse wave_lse(Lse p) {
    // butterfly over the wave with DPP-free shuffles (ds_swizzle/bpermute)
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        Lse q;
        q.m = __shfl_xor(p.m, off, 64);
        q.s = __shfl_xor(p.s, off, 64);
        p = lse_merge(p, q);
    }
    return p;
}

__device__ __forceinline__ float update_potential(float lse, float log_marg, float old,
                                                  float damp, bool unbalanced) {
    if (!isfinite(lse))
        return old;
    const float diff = log_marg - lse;
    return unbalanced ? damp * diff : diff;
}

// ---- row sweep: log_u ----------------------------------------------------------

// One wave per row: lse_c = LSE_j(K[i, j] + log_v[j]), then the log_u update.
__global__ void __launch_bounds__(kRowBlock)
sk_row_sweep(const float *__restrict__ K, const float *__restrict__ log_v,
             const float *__restrict__ log_mu, const uint8_t *__restrict__ inf_row,
             float *__restrict__ log_u, int64_t B, int64_t N, int64_t M, float damp,
             int unbalanced) {
    const int64_t r = (int64_t)blockIdx.x * (kRowBlock / 64) + threadIdx.x / 64;
    if (r >= B * N)
        return;
    const int64_t b = r / N;
    const int lane = lane_id();
    if (inf_row[r])
        return;  // lse = -inf: log_u keeps its value
    const float *row = K + r * M;
    const float *lv = log_v + b * M;
    Lse acc{-f_inf(), 0.f};
    if ((M & 3) == 0) {
        const float4 *row4 = reinterpret_cast<const float4 *>(row);
        const float4 *lv4 = reinterpret_cast<const float4 *>(lv);
        const int64_t m4 = M / 4;
        for (int64_t q = lane; q < m4; q += 64) {
            const float4 k = row4[q];
            const float4 v = lv4[q];
            const float t[4] = {k.x + v.x, k.y + v.y, k.z + v.z, k.w + v.w};
            lse_push<4>(acc, t);
        }
    } else {
        for (int64_t j = lane; j < M; j += 64) {
            const float t[1] = {row[j] + lv[j]};
            lse_push<1>(acc, t);
        }
    }
    acc = wave_lse(acc);
    if (lane == 0) {
        const float lse = lse_value(acc);
        log_u[r] = update_potential(lse, log_mu[r], log_u[r], damp, unbalanced != 0);
    }
}

// ---- column sweep: log_v -------------------------------------------------------

// grid (n_strip, n_chunk, B); thread t owns columns strip*1024 + 4t .. +3 and
// folds rows [chunk*R, chunk*R + R) into per-column partial pairs.
__global__ void __launch_bounds__(kColBlock)
sk_col_partial(const float *__restrict__ K, const float *__restrict__ log_u,
               float2 *__restrict__ colpart, int64_t N, int64_t M, int rows_per_chunk,
               int n_chunk) {
    const int strip = blockIdx.x, chunk = blockIdx.y;
    const int64_t b = blockIdx.z;
    const int64_t j0 = (int64_t)strip * kColStrip + 4 * threadIdx.x;
    const int64_t i0 = (int64_t)chunk * rows_per_chunk;
    const int64_t i1 = (i0 + rows_per_chunk < N) ? i0 + rows_per_chunk : N;
    const float *Kb = K + b * N * M;
    const float *lu = log_u + b * N;
    Lse acc[4] = {{-f_inf(), 0.f}, {-f_inf(), 0.f}, {-f_inf(), 0.f}, {-f_inf(), 0.f}};
    if (j0 < M) {
        if ((M & 3) == 0) {
            for (int64_t i = i0; i < i1; ++i) {
                const float4 k = *reinterpret_cast<const float4 *>(Kb + i * M + j0);
                const float u = lu[i];
                const float t0[1] = {k.x + u}, t1[1] = {k.y + u}, t2[1] = {k.z + u},
                            t3[1] = {k.w + u};
                lse_push<1>(acc[0], t0);
                lse_push<1>(acc[1], t1);
                lse_push<1>(acc[2], t2);
                lse_push<1>(acc[3], t3);
            }
        } else {
            for (int64_t i = i0; i < i1; ++i) {
                const float u = lu[i];
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (j0 + c < M) {
                        const float t[1] = {Kb[i * M + j0 + c] + u};
                        lse_push<1>(acc[c], t);
                    }
            }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (j0 + c < M)
                colpart[(b * n_chunk + chunk) * M + j0 + c] = make_float2(acc[c].m, acc[c].s);
    }
}

// One thread per (b, j): merge the chunk partials, then the log_v update.
__global__ void __launch_bounds__(kMapBlock)
sk_col_merge(const float2 *__restrict__ colpart, const float *__restrict__ log_nu,
             const uint8_t *__restrict__ inf_col, float *__restrict__ log_v, int64_t B,
             int64_t M, int n_chunk, float damp, int unbalanced) {
    const int64_t t = (int64_t)blockIdx.x * kMapBlock + threadIdx.x;
    if (t >= B * M)
        return;
    if (inf_col[t])
        return;
    const int64_t b = t / M, j = t % M;
    Lse acc{-f_inf(), 0.f};
    for (int c = 0; c < n_chunk; ++c) {
        const float2 p = colpart[(b * n_chunk + c) * M + j];
        acc = lse_merge(acc, Lse{p.x, p.y});
    }
    const float lse = lse_value(acc);
    log_v[t] = update_potential(lse, log_nu[t], log_v[t], damp, unbalanced != 0);
}

// ---- final plan ----------------------------------------------------------------

// log_plan[b,i,j] = (log_u[b,i] + (-C[b,i,j] / e)) + log_v[b,j]
__global__ void __launch_bounds__(kMapBlock)
sk_plan(const float *__restrict__ C, const float *__restrict__ log_u,
        const float *__restrict__ log_v, float *__restrict__ plan, int64_t B, int64_t N,
        int64_t M, float eps) {
    const int64_t n = B * N * M;
    const int64_t stride = (int64_t)gridDim.x * kMapBlock;
    for (int64_t k = (int64_t)blockIdx.x * kMapBlock + threadIdx.x; k < n; k += stride) {
        const int64_t row = k / M;
        const int64_t j = k - row * M;
        const int64_t b = row / N;
        plan[k] = (log_u[row] + (-C[k] / eps)) + log_v[b * M + j];
    }
}

int grid_for(int64_t n, int block, int cap) {
    int64_t g = (n + block - 1) / block;
    if (g < 1)
        g = 1;
    return (int)(g > cap ? cap : g);
}

} // namespace
} // namespace tmamd

using namespace tmamd;

extern "C" size_t tm_sinkhorn_workspace_bytes(int64_t B, int64_t N, int64_t M) {
    if (B <= 0 || N <= 0 || M <= 0)
        return 256;
    return make_layout(B, N, M).total;
}

extern "C" int tm_sinkhorn_f32(const float *cost, const float *a, const float *b, int64_t B,
                               int64_t N, int64_t M, const double *eps_sched, int32_t n_iter,
                               double rho, float *log_plan, float *log_u, float *log_v,
                               void *workspace, size_t workspace_bytes, hipStream_t stream) {
    if (B < 0 || N < 0 || M < 0 || n_iter < 1 || eps_sched == nullptr)
        return TM_ERR_INVALID_ARGUMENT;
    for (int32_t s = 0; s < n_iter; ++s)
        if (!(eps_sched[s] > 0.0))
            return TM_ERR_INVALID_ARGUMENT;
    if (B == 0 || N == 0 || M == 0)
        return TM_OK;
    const SinkhornLayout L = make_layout(B, N, M);
    if (workspace == nullptr || workspace_bytes < L.total)
        return TM_ERR_WORKSPACE;
    if (L.n_strip > 65535 || L.n_chunk > 65535 || B > 65535)
        return TM_ERR_UNSUPPORTED_SHAPE;
    char *ws = static_cast<char *>(workspace);
    float *K = reinterpret_cast<float *>(ws + L.off_k);
    float *log_mu = reinterpret_cast<float *>(ws + L.off_logmu);
    float *log_nu = reinterpret_cast<float *>(ws + L.off_lognu);
    uint8_t *inf_row = reinterpret_cast<uint8_t *>(ws + L.off_infrow);
    uint8_t *inf_col = reinterpret_cast<uint8_t *>(ws + L.off_infcol);
    float2 *colpart = reinterpret_cast<float2 *>(ws + L.off_colpart);
    const bool unbalanced = rho > 0.0;
    const int64_t nK = B * N * M;

#define TM_LAUNCH(...)                                                                    \
    do {                                                                                  \
        hipLaunchKernelGGL(__VA_ARGS__);                                                  \
        if (hipGetLastError() != hipSuccess)                                              \
            return TM_ERR_LAUNCH;                                                         \
    } while (0)

    TM_LAUNCH(sk_log_marginal, dim3(grid_for(B * N, kMapBlock, 1 << 30)), dim3(kMapBlock), 0,
              stream, a, log_mu, B * N);
    TM_LAUNCH(sk_log_marginal, dim3(grid_for(B * M, kMapBlock, 1 << 30)), dim3(kMapBlock), 0,
              stream, b, log_nu, B * M);
    TM_LAUNCH(sk_fill, dim3(grid_for(B * N, kMapBlock, 1 << 30)), dim3(kMapBlock), 0, stream,
              log_u, B * N, 0.f);
    TM_LAUNCH(sk_fill, dim3(grid_for(B * M, kMapBlock, 1 << 30)), dim3(kMapBlock), 0, stream,
              log_v, B * M, 0.f);
    TM_LAUNCH(sk_inf_rows, dim3(grid_for(B * N, kRowBlock / 64, 1 << 30)), dim3(kRowBlock), 0,
              stream, cost, inf_row, B * N, M);
    TM_LAUNCH(sk_inf_cols, dim3(grid_for(B * M, kMapBlock, 1 << 30)), dim3(kMapBlock), 0,
              stream, cost, inf_col, B, N, M);

    const int map_grid = grid_for(nK / 4 + 1, kMapBlock, 8192);
    float cur_eps = -1.f;
    for (int32_t s = 0; s < n_iter; ++s) {
        const float e = (float)eps_sched[s];
        if (e != cur_eps) {
            TM_LAUNCH(sk_log_kernel, dim3(map_grid), dim3(kMapBlock), 0, stream, cost, K, nK, e);
            cur_eps = e;
        }
        const float damp = unbalanced ? (float)(1.0 / (1.0 + eps_sched[s] / rho)) : 1.f;
        TM_LAUNCH(sk_row_sweep, dim3(grid_for(B * N, kRowBlock / 64, 1 << 30)), dim3(kRowBlock),
                  0, stream, K, log_v, log_mu, inf_row, log_u, B, N, M, damp,
                  unbalanced ? 1 : 0);
        TM_LAUNCH(sk_col_partial, dim3(L.n_strip, L.n_chunk, (unsigned)B), dim3(kColBlock), 0,
                  stream, K, log_u, colpart, N, M, L.rows_per_chunk, L.n_chunk);
        TM_LAUNCH(sk_col_merge, dim3(grid_for(B * M, kMapBlock, 1 << 30)), dim3(kMapBlock), 0,
                  stream, colpart, log_nu, inf_col, log_v, B, M, L.n_chunk, damp,
                  unbalanced ? 1 : 0);
    }
    if (log_plan != nullptr) {
        const float ef = (float)eps_sched[n_iter - 1];
        TM_LAUNCH(sk_plan, dim3(grid_for(nK, kMapBlock, 8192)), dim3(kMapBlock), 0, stream,
                  cost, log_u, log_v, log_plan, B, N, M, ef);
    }
#undef TM_LAUNCH
    return TM_OK;
}
