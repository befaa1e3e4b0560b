// sinkhorn64.hip -- log-domain Sinkhorn in float64 for gfx950.
//
// The reference iterates in the cost's dtype (transport/matrix/
// _log_sinkhorn.py:184,191; _unbalanced_sinkhorn.py:60,67), so a float64 cost
// gets float64 arithmetic throughout.  This is the plain two-sweep form of
// the same iteration (the float32 path's one-read fused step relies on
// float32-specific shifts): per step, one block per row for the row
// logsumexp and log_u, then column strips for the column logsumexp and
// log_v, each with the reference's two-pass shift rule (the maximum, or 0
// when it is +-inf) and its `isfinite` keep-previous rule.
//   log_kernel = -cost / eps           _log_sinkhorn.py:194 (IEEE division)
//   fully +inf rows / columns          _log_sinkhorn.py:33-46 (their potential
//                                       keeps its value: the -80 stand-in's
//                                       LSE is overwritten by -inf)
//   damping 1 / (1 + eps / rho)        _unbalanced_sinkhorn.py:71
//   plan (log_u + K) + log_v           _log_sinkhorn.py:217
// The caller validates the cost (no NaN / -inf) and fuses any mask into it.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/torchmatch_amd.h"

namespace {

constexpr int kThreads = 256;      // row block / column-strip block
constexpr int kStrip = 64;         // columns per strip
constexpr int kGroups = kThreads / kStrip;

struct Layout64 {
    size_t off_k, off_logmu, off_lognu, off_infrow, off_infcol, total;
};

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

Layout64 layout64(int64_t B, int64_t N, int64_t M) {
    Layout64 L{};
    size_t off = 0;
    L.off_k = off;
    off = align256(off + sizeof(double) * (size_t)(B * N * M));
    L.off_logmu = off;
    off = align256(off + sizeof(double) * (size_t)(B * N));
    L.off_lognu = off;
    off = align256(off + sizeof(double) * (size_t)(B * M));
    L.off_infrow = off;
    off = align256(off + (size_t)(B * N));
    L.off_infcol = off;
    off = align256(off + (size_t)(B * M));
    L.total = off;
    return L;
}

__device__ __forceinline__ double shift_of(double m) { return isinf(m) ? 0.0 : m; }

// Block-wide max / sum over kThreads lanes (uniform result).
__device__ double block_max(double x, double *red) {
    red[threadIdx.x] = x;
    __syncthreads();
    for (int s = kThreads / 2; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s)
            red[threadIdx.x] = fmax(red[threadIdx.x], red[threadIdx.x + s]);
        __syncthreads();
    }
    const double r = red[0];
    __syncthreads();
    return r;
}

__device__ double block_sum(double x, double *red) {
    red[threadIdx.x] = x;
    __syncthreads();
    for (int s = kThreads / 2; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s)
            red[threadIdx.x] += red[threadIdx.x + s];
        __syncthreads();
    }
    const double r = red[0];
    __syncthreads();
    return r;
}

__global__ void sk64_log_marginal(const double *__restrict__ m, double *__restrict__ out,
                                  int64_t n) {
    for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < n;
         k += (int64_t)gridDim.x * blockDim.x)
        out[k] = log(m[k]);
}

__global__ void sk64_fill(double *__restrict__ x, int64_t n, double v) {
    for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < n;
         k += (int64_t)gridDim.x * blockDim.x)
        x[k] = v;
}

// K = -C / eps, and (first call) the fully +inf row / column flags.
__global__ void sk64_log_kernel(const double *__restrict__ c, double *__restrict__ K,
                                int64_t n, double eps) {
    for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < n;
         k += (int64_t)gridDim.x * blockDim.x)
        K[k] = -c[k] / eps;
}

__global__ void __launch_bounds__(kThreads)
sk64_row_flags(const double *__restrict__ c, uint8_t *__restrict__ inf_row, int64_t rows,
               int64_t M) {
    __shared__ int any_finite;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        if (threadIdx.x == 0)
            any_finite = 0;
        __syncthreads();
        const double *row = c + r * M;
        int f = 0;
        for (int64_t j = threadIdx.x; j < M; j += kThreads)
            f |= (row[j] != INFINITY) ? 1 : 0;
        if (f)
            atomicOr(&any_finite, 1);
        __syncthreads();
        if (threadIdx.x == 0)
            inf_row[r] = any_finite ? 0 : 1;
        __syncthreads();
    }
}

__global__ void sk64_col_flags(const double *__restrict__ c, uint8_t *__restrict__ inf_col,
                               int64_t B, int64_t N, int64_t M) {
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < B * M;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t b = t / M, j = t % M;
        const double *col = c + b * N * M + j;
        uint8_t all_inf = 1;
        for (int64_t i = 0; i < N; ++i)
            if (col[i * M] != INFINITY) {
                all_inf = 0;
                break;
            }
        inf_col[t] = all_inf;
    }
}

// Row half-step: lse_j(K + log_v) per row, then log_u (keep-previous rule).
__global__ void __launch_bounds__(kThreads)
sk64_row(const double *__restrict__ K, const double *__restrict__ log_v,
         const double *__restrict__ log_mu, const uint8_t *__restrict__ inf_row,
         double *__restrict__ log_u, int64_t B, int64_t N, int64_t M, double damp,
         int unbalanced) {
    __shared__ double red[kThreads];
    for (int64_t r = blockIdx.x; r < B * N; r += gridDim.x) {
        if (inf_row[r])
            continue;  // uniform per block: the potential keeps its value
        const int64_t b = r / N;
        const double *row = K + r * M;
        const double *lv = log_v + b * M;
        double m = -INFINITY;
        for (int64_t j = threadIdx.x; j < M; j += kThreads)
            m = fmax(m, row[j] + lv[j]);
        const double sh = shift_of(block_max(m, red));
        double s = 0.0;
        for (int64_t j = threadIdx.x; j < M; j += kThreads)
            s += exp((row[j] + lv[j]) - sh);
        const double lse = log(block_sum(s, red)) + sh;
        if (threadIdx.x == 0 && isfinite(lse)) {
            const double diff = log_mu[r] - lse;
            log_u[r] = unbalanced ? damp * diff : diff;
        }
    }
}

// Column half-step: lse_i(K + log_u) per column (64-column strips, four row
// groups), then log_v (keep-previous rule).  Blocks stride over the
// (batch, strip) pairs on gridDim.x, so the batch size has no grid limit.
__global__ void __launch_bounds__(kThreads)
sk64_col(const double *__restrict__ K, const double *__restrict__ log_u,
         const double *__restrict__ log_nu, const uint8_t *__restrict__ inf_col,
         double *__restrict__ log_v, int64_t B, int64_t N, int64_t M, double damp,
         int unbalanced) {
    __shared__ double part[kGroups][kStrip];
    const int lc = threadIdx.x % kStrip, g = threadIdx.x / kStrip;
    const int64_t strips = (M + kStrip - 1) / kStrip;
    for (int64_t task = blockIdx.x; task < B * strips; task += gridDim.x) {
        const int64_t b = task / strips;
        const int64_t j = (task - b * strips) * kStrip + lc;
        const bool live = j < M;
        const double *Kb = K + b * N * M;
        const double *lu = log_u + b * N;
        double m = -INFINITY;
        if (live)
            for (int64_t i = g; i < N; i += kGroups)
                m = fmax(m, Kb[i * M + j] + lu[i]);
        part[g][lc] = m;
        __syncthreads();
        double mm = part[0][lc];
        for (int k = 1; k < kGroups; ++k)
            mm = fmax(mm, part[k][lc]);
        const double sh = shift_of(mm);
        __syncthreads();
        double s = 0.0;
        if (live)
            for (int64_t i = g; i < N; i += kGroups)
                s += exp((Kb[i * M + j] + lu[i]) - sh);
        part[g][lc] = s;
        __syncthreads();
        if (g == 0 && live) {
            double ss = part[0][lc];
            for (int k = 1; k < kGroups; ++k)
                ss += part[k][lc];
            const double lse = log(ss) + sh;
            const int64_t t = b * M + j;
            if (!inf_col[t] && isfinite(lse)) {
                const double diff = log_nu[t] - lse;
                log_v[t] = unbalanced ? damp * diff : diff;
            }
        }
        __syncthreads();  // part[] is written again by the next task
    }
}

__global__ void sk64_plan(const double *__restrict__ K, const double *__restrict__ log_u,
                          const double *__restrict__ log_v, double *__restrict__ plan,
                          int64_t B, int64_t N, int64_t M) {
    const int64_t n = B * N * M;
    for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < n;
         k += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = k / M;           // b * N + i
        const int64_t b = r / N, j = k % M;
        plan[k] = (log_u[r] + K[k]) + log_v[b * M + j];
    }
}

unsigned grid_for(int64_t n, int per, int64_t cap) {
    int64_t g = (n + per - 1) / per;
    if (g < 1)
        g = 1;
    return (unsigned)(g > cap ? cap : g);
}

#define TM64_LAUNCH(kernel, grid, block, stream, ...)                                   \
    do {                                                                                \
        hipLaunchKernelGGL(kernel, grid, block, 0, stream, __VA_ARGS__);                \
        if (hipGetLastError() != hipSuccess)                                            \
            return TM_ERR_LAUNCH;                                                       \
    } while (0)

} // namespace

extern "C" size_t tm_sinkhorn_f64_workspace_bytes(int64_t B, int64_t N, int64_t M) {
    if (B < 0 || N < 0 || M < 0)
        return 0;
    return layout64(B, N, M).total;
}

extern "C" int tm_sinkhorn_f64(const double *cost, const double *a, const double *b, int64_t B,
                               int64_t N, int64_t M, const double *eps_sched, int32_t n_iter,
                               double rho, double *log_plan, double *log_u, double *log_v,
                               void *workspace, size_t workspace_bytes, hipStream_t stream) {
    if (B < 0 || N < 0 || M < 0 || n_iter < 1 || eps_sched == nullptr)
        return TM_ERR_INVALID_ARGUMENT;
    for (int32_t s = 0; s < n_iter; ++s)
        if (!(eps_sched[s] > 0.0))
            return TM_ERR_INVALID_ARGUMENT;
    if (B == 0)
        return TM_OK;
    if ((N > 0 && log_u == nullptr) || (M > 0 && log_v == nullptr))
        return TM_ERR_INVALID_ARGUMENT;
    if (N > 0)
        TM64_LAUNCH(sk64_fill, dim3(grid_for(B * N, 256, 1 << 16)), dim3(256), stream, log_u,
                    B * N, 0.0);
    if (M > 0)
        TM64_LAUNCH(sk64_fill, dim3(grid_for(B * M, 256, 1 << 16)), dim3(256), stream, log_v,
                    B * M, 0.0);
    if (N == 0 || M == 0)
        return TM_OK;  // no pair: the potentials keep their start value
    if (cost == nullptr || a == nullptr || b == nullptr)
        return TM_ERR_INVALID_ARGUMENT;
    const Layout64 L = layout64(B, N, M);
    if (workspace == nullptr || workspace_bytes < L.total)
        return TM_ERR_WORKSPACE;
    char *ws = static_cast<char *>(workspace);
    double *K = reinterpret_cast<double *>(ws + L.off_k);
    double *log_mu = reinterpret_cast<double *>(ws + L.off_logmu);
    double *log_nu = reinterpret_cast<double *>(ws + L.off_lognu);
    uint8_t *inf_row = reinterpret_cast<uint8_t *>(ws + L.off_infrow);
    uint8_t *inf_col = reinterpret_cast<uint8_t *>(ws + L.off_infcol);
    const int64_t nK = B * N * M;
    const dim3 map_grid(grid_for(nK, 256, 1 << 16));
    TM64_LAUNCH(sk64_log_marginal, dim3(grid_for(B * N, 256, 1 << 16)), dim3(256), stream, a,
                log_mu, B * N);
    TM64_LAUNCH(sk64_log_marginal, dim3(grid_for(B * M, 256, 1 << 16)), dim3(256), stream, b,
                log_nu, B * M);
    TM64_LAUNCH(sk64_row_flags, dim3(grid_for(B * N, 1, 1 << 16)), dim3(kThreads), stream, cost,
                inf_row, B * N, M);
    TM64_LAUNCH(sk64_col_flags, dim3(grid_for(B * M, 256, 1 << 16)), dim3(256), stream, cost,
                inf_col, B, N, M);
    const bool unbalanced = rho > 0.0;
    const dim3 row_grid(grid_for(B * N, 1, 1 << 16));
    const dim3 col_grid(grid_for(B * ((M + kStrip - 1) / kStrip), 1, 1 << 16));
    double cur = -1.0;
    for (int32_t s = 0; s < n_iter; ++s) {
        const double e = eps_sched[s];
        if (e != cur) {
            TM64_LAUNCH(sk64_log_kernel, map_grid, dim3(256), stream, cost, K, nK, e);
            cur = e;
        }
        const double damp = unbalanced ? 1.0 / (1.0 + e / rho) : 1.0;
        TM64_LAUNCH(sk64_row, row_grid, dim3(kThreads), stream, K, log_v, log_mu, inf_row,
                    log_u, B, N, M, damp, unbalanced ? 1 : 0);
        TM64_LAUNCH(sk64_col, col_grid, dim3(kThreads), stream, K, log_u, log_nu, inf_col,
                    log_v, B, N, M, damp, unbalanced ? 1 : 0);
    }
    if (log_plan != nullptr)
        TM64_LAUNCH(sk64_plan, map_grid, dim3(256), stream, K, log_u, log_v, log_plan, B, N, M);
    return TM_OK;
}
