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
// HBM layout (row-major, resident for the whole call):
//   K        (B, N, M)  float32 log kernel, rewritten only when the schedule's
//                       epsilon changes (once for a constant schedule): -C/e
//                       for the two-sweep step, -C*log2(e)/e for the fused one
//   log_u/v  (B, N) / (B, M) the caller's float32 outputs, written every step
//   colpart  (B, n_chunk, M) column partials of row chunks: float sums (fused
//                       step) or float2 (max, sum) pairs (exact fused step,
//                       two-sweep column sweep with chunked rows)
//   fused step state: float64 potentials and log marginals, the potentials
//                       scaled by log2(e) in float32 with their rounding
//                       weights, each row's base-2 LSE of the previous step
//
// One step, in one of two forms:
//   fused (sk_fused_step + sk_col_merge_blk; 128 <= M <= 16384, M % 4 == 0):
//     K is read once.  Each row's LSE is reduced from registers, its log_u
//     updated in float64, and the row's terms, times one factor of the row,
//     are added into per-column sums; the merge adds the chunks' sums and
//     recomputes exactly any column whose total left the accepted window.
//     B*N*M*4 algorithmic bytes.
//   two-sweep (sk_row_sweep* + sk_col_sweep [+ sk_col_merge]): a row sweep
//     and a column sweep each read K, 2 * B*N*M*4 bytes.
//
// Row sweep: rows of up to 2048 columns belong to one wave each, and each
// is an exact two-pass LSE over registers (max, then sum of exp); longer rows
// are split over the eight waves of a block in 1024-column chunks, whose
// (max, sum) pairs merge in LDS.  Column sweep: a block owns a column strip over a
// chunk of rows; 16 threads span a 64-column strip (8 a 32-column one) with
// float4 loads, 16 (32) row groups fold rows online (one rescale per group of
// U rows), and an LDS merge of the row groups yields the column LSE (or a
// partial when rows are chunked).
// exp / log run on the native v_exp_f32 / v_log_f32 (base 2).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "jv_batch.h"
#include "wave.h"

namespace tmamd {
namespace {

constexpr int kMapBlock = 256;
constexpr int kRowWaves = 4;          // waves per row-sweep block
constexpr int kRowsPerWave = 1;       // rows per wave (occupancy beats log_v reuse)
constexpr int kRowNV = 8;             // float4 per lane per row chunk (2048 cols)
constexpr int kColThreads = 256;      // column-sweep block: strip threads x row groups
constexpr int kColStrip = 64;         // strip width (columns): 16 threads x 16 row groups
constexpr int kColStripNarrow = 32;   // narrow strip: 8 threads x 32 row groups
constexpr int64_t kColNarrowBlocks = 4 * 256;  // narrow strips when they fill this many
constexpr int64_t kColBlocksTarget = 5 * 256;  // column-sweep blocks to aim for
constexpr int kColU = 8;              // rows per group fold
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// 1 / kLog2e as an unevaluated sum hi + lo (hi is the float nearest ln 2).  The
// one-read step works in base-2 units, y = kLog2e * (K + log_v), and converts
// each LSE back with this pair: kLn2 * kLog2e = 1 - 1.06e-8, so converting
// with kLn2 alone scales every update by that factor, a bias that the
// potentials' neutral mode (log_u + c, log_v - c) accumulates step after step
// (C4: 3.4e-5 in log_u after 200 iterations against 1.8e-6 for the float32
// reference); the pair leaves 2e-16.
constexpr float kInvLog2eHi = 0.693147182464599609375f;   // 0x3f317218
constexpr float kInvLog2eLo = 7.348693209507928e-09f;     // 0x31fc7fca

__device__ __forceinline__ float f_inf() { return __int_as_float(0x7f800000); }

// log2 e and ln 2 as hi + lo float pairs (hi = the float constants above):
// the two-sweep step's exp and log go through base 2 on every element and
// row, and a constant's rounding would bias each update by ~1e-8 relative,
// which the potentials' neutral mode accumulates over the iterations
constexpr float kLog2eLo = 1.925963033500011e-08f;  // 0x32a57060
constexpr float kLn2Lo = -1.9046542121259336e-09f;  // 0xb102e308

// e^(x) for x <= 0 (or -inf) on the native base-2 unit
__device__ __forceinline__ float exp_nonpos(float x) {
    return __builtin_amdgcn_exp2f(fmaf(x, kLog2e, x * kLog2eLo));
}
// natural log of s >= 0 (log(0) = -inf)
__device__ __forceinline__ float ln(float s) {
    const float l2 = __builtin_amdgcn_logf(s);
    return fmaf(l2, kLn2, l2 * kLn2Lo);
}

// natural-unit LSE from a base-2 LSE of kLog2e-scaled values
__device__ __forceinline__ float ln_of_lse2(float l2) {
    return fmaf(l2, kInvLog2eHi, l2 * kInvLog2eLo);
}

__device__ __forceinline__ float lse_shift(float m) { return isinf(m) ? 0.f : m; }

struct Lse {
    float m;  // running max (may be -inf)
    float s;  // sum of exp(t - shift(m))
};

__device__ __forceinline__ Lse lse_merge(Lse p, Lse q) {
    const float m = fmaxf(p.m, q.m);
    const float sh = lse_shift(m);
    const float a = (p.s == 0.f) ? 0.f : p.s * exp_nonpos(lse_shift(p.m) - sh);
    const float c = (q.s == 0.f) ? 0.f : q.s * exp_nonpos(lse_shift(q.m) - sh);
    return Lse{m, a + c};
}

__device__ __forceinline__ float lse_value(Lse p) { return ln(p.s) + lse_shift(p.m); }

__device__ __forceinline__ float wave_sum(float x) {
    x += __shfl_xor(x, 1, 64);
    x += __shfl_xor(x, 2, 64);
    x += __shfl_xor(x, 4, 64);
    x += __shfl_xor(x, 8, 64);
    x += __shfl_xor(x, 16, 64);
    x += __shfl_xor(x, 32, 64);
    return x;
}

__device__ __forceinline__ Lse wave_lse(Lse p) {
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

// ---- workspace ----------------------------------------------------------------

struct SinkhornLayout {
    int64_t B, N, M;
    int n_chunk, rows_per_chunk, n_strip, strip;
    int fused;                   // FusedVariant of sk_fused_step, 0: two-sweep step
    int fz_chunk, fz_rows;       // its row chunks per batch and rows per chunk
    int fz_interleave;           // chunks take every n_chunk-th row (else a range)
    size_t off_k, off_logmu, off_lognu, off_infrow, off_infcol, off_colpart, off_lse2row,
        off_stats, total;
    // float64 state of the fused step: the potentials, the marginals' logs,
    // and the potentials scaled by kLog2e in float32 (what the element
    // loops add), B*N / B*M each
    size_t off_lu64, off_lv64, off_mu64, off_nu64, off_lu2, off_lv2;
    // per-column weights 2^(lv2 rounding residual), float32, B*M
    size_t off_lvw;
};

__host__ __device__ inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// sk_fused_step instantiations: (W waves per row, RW row groups, NV float4
// per lane), chosen by row length; resident blocks per CU from their VGPR and
// LDS use (hipcc's resource report for the non-EXACT instances: 1x4x4 104
// VGPRs, 1x4x8 199, 2x1x8 and 4x1x8 190, 8x1x8 226, 16x1x4 122; LDS 12 / 24 /
// 16 / 32 / 64 / 65 KiB; the short-row shapes 47 and 67 VGPRs).  Rows
// longer than 8192 columns take 16 waves of 1024 columns, one block per CU
// (four waves per SIMD at 122 VGPRs; 8 waves of 2048 columns measured
// slower).
enum FusedVariant {
    kFzNone = 0, kFz1x4x4, kFz1x4x8, kFz2x1x8, kFz4x1x8, kFz8x1x8, kFz16x1x4, kFz1x4x1, kFz1x4x2
};
// K sizes above which the fused step streams K with non-temporal loads.
constexpr size_t kNonTemporalBytes = (size_t)384 << 20;

struct FusedShape {
    int W, RW, NV, blocks_per_cu;
};
constexpr FusedShape kFusedShapes[] = {
    {0, 0, 0, 0}, {1, 4, 4, 4}, {1, 4, 8, 2}, {2, 1, 8, 4}, {4, 1, 8, 2}, {8, 1, 8, 1},
    {16, 1, 4, 1}, {1, 4, 1, 8}, {1, 4, 2, 8},
};
constexpr int kFusedMinRowsPerWave = 8;

void choose_fused(SinkhornLayout &L) {
    L.fused = kFzNone;
    L.fz_chunk = L.fz_rows = 0;
    const int64_t M = L.M;
    if (M % 4 != 0 || M < 128 || M > 16384)
        return;
    L.fused = M <= 256    ? kFz1x4x1
              : M <= 512  ? kFz1x4x2
              : M <= 1024 ? kFz1x4x4
              : M <= 2048 ? kFz1x4x8
              : M <= 4096 ? kFz2x1x8
              : M <= 8192 ? kFz4x1x8
                          : kFz16x1x4;
    if (const char *env = getenv("TORCHMATCH_AMD_SINKHORN_FUSED")) {
        // "0": the two-sweep step; "8x1x8": that long-row shape
        if (strcmp(env, "0") == 0)
            L.fused = kFzNone;
        else if (strcmp(env, "8x1x8") == 0 && M > 8192)
            L.fused = kFz8x1x8;
        if (L.fused == kFzNone)
            return;
    }
    const FusedShape &f = kFusedShapes[L.fused];
    // one resident round of blocks over the 256 CUs, each wave >= 8 rows
    int64_t chunks = (256 * (int64_t)f.blocks_per_cu) / L.B;
    const int64_t max_chunks = L.N / ((int64_t)f.RW * kFusedMinRowsPerWave);
    if (chunks > max_chunks)
        chunks = max_chunks;
    if (chunks < 1)
        chunks = 1;
    L.fz_rows = (int)((L.N + chunks - 1) / chunks);
    L.fz_chunk = (int)((L.N + L.fz_rows - 1) / L.fz_rows);
    // rows split over several waves (one block per CU): blocks march through
    // the rows side by side (measured faster on C5); rows of one wave: each
    // block streams its own range (faster on C4)
    L.fz_interleave = f.W > 1;
}

SinkhornLayout make_layout(int64_t B, int64_t N, int64_t M) {
    SinkhornLayout L{};
    L.B = B;
    L.N = N;
    L.M = M;
    // 32-column strips when they alone give the column sweep about four
    // blocks per CU (no row chunks, so no merge pass: C4 runs 81 us per
    // iteration instead of 83), else 64-column strips split into row chunks
    // until there are about five blocks per CU (68 VGPRs allow seven; five
    // measured best), keeping >= 256 rows per chunk
    L.strip = B * ((M + kColStripNarrow - 1) / kColStripNarrow) >= kColNarrowBlocks
                  ? kColStripNarrow
                  : kColStrip;
    L.n_strip = (int)((M + L.strip - 1) / L.strip);
    const int64_t blocks = B * L.n_strip;
    int64_t chunks = kColBlocksTarget / blocks;
    if (chunks < 1)
        chunks = 1;
    while (chunks > 1 && N / chunks < 256)
        --chunks;
    L.n_chunk = (int)chunks;
    L.rows_per_chunk = (int)((N + chunks - 1) / chunks);
    choose_fused(L);
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
    {
        int64_t parts = L.n_chunk > 1 ? L.n_chunk : 0;
        if (L.fused && L.fz_chunk > parts)
            parts = L.fz_chunk;
        off = align_up(off + sizeof(float2) * (size_t)B * (size_t)parts * (size_t)M, 256);
    }
    L.off_lse2row = off;
    if (L.fused)
        off = align_up(off + sizeof(float) * (size_t)(B * N), 256);
    L.off_lu64 = off;
    if (L.fused)
        off = align_up(off + sizeof(double) * (size_t)(B * N), 256);
    L.off_lv64 = off;
    if (L.fused)
        off = align_up(off + sizeof(double) * (size_t)(B * M), 256);
    L.off_mu64 = off;
    if (L.fused)
        off = align_up(off + sizeof(double) * (size_t)(B * N), 256);
    L.off_nu64 = off;
    if (L.fused)
        off = align_up(off + sizeof(double) * (size_t)(B * M), 256);
    L.off_lu2 = off;
    if (L.fused)
        off = align_up(off + sizeof(float) * (size_t)(B * N), 256);
    L.off_lv2 = off;
    if (L.fused)
        off = align_up(off + sizeof(float) * (size_t)(B * M), 256);
    L.off_lvw = off;
    if (L.fused)
        off = align_up(off + sizeof(float) * (size_t)(B * M), 256);
    L.off_stats = off;
    off += 256;
    L.total = off;
    return L;
}

// ---- preparation: one pass over the cost ----------------------------------------

constexpr int kPrepWaves = 4;                                // waves per prepare block
constexpr int kPrepRowsPerWave = 8;                          // rows a wave keeps in flight
constexpr int kPrepRows = kPrepWaves * kPrepRowsPerWave;     // rows per block and group
constexpr uint32_t kFlagNan = TM_SK_FLAG_NAN, kFlagNegInf = TM_SK_FLAG_NEG_INF;
constexpr uint32_t kFlagANeg = TM_SK_FLAG_A_NEG, kFlagBNeg = TM_SK_FLAG_B_NEG;

// Order-preserving key of a float: f < g  <=>  key(f) < key(g); every float
// that is not a negative NaN maps above 0, so 0 means "no value".
__device__ __forceinline__ uint32_t order_key(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// K = -C'/e (IEEE division, as torch's `-cost / step_eps` in float32), where
// C' = C, or with a keep mask C' = keep ? C : +inf (torch's
// `cost.masked_fill(~mask, inf)`), so masked pairs hold -inf.  Float4 steps
// when `vec` (C and K 16-byte aligned, keep 4-byte aligned), else scalar.
// One element of K from C': -C'/e (float32 IEEE division, the reference's
// expression) when s2 == 0, else C' * s2 rounded once to float32 with
// s2 = -log2(e)/e in float64: the fused step's base-2 log kernel, in which
// 2^(K + p) is exactly e^(-C'/e + p/log2(e)) up to the one rounding of K.
__device__ __forceinline__ float k_of(float c, float e, double s2) {
    return s2 != 0.0 ? (float)((double)c * s2) : -c / e;
}

template <bool MASK>
__global__ void __launch_bounds__(kMapBlock)
sk_log_kernel(const float *__restrict__ C, const uint8_t *__restrict__ keep,
              float *__restrict__ K, int64_t n, float eps, double s2, int vec) {
    const int64_t stride = (int64_t)gridDim.x * kMapBlock;
    const int64_t n4 = vec ? n / 4 : 0;
    const float4 *c4 = reinterpret_cast<const float4 *>(C);
    const uint32_t *kp4 = reinterpret_cast<const uint32_t *>(keep);
    float4 *k4 = reinterpret_cast<float4 *>(K);
    for (int64_t k = (int64_t)blockIdx.x * kMapBlock + threadIdx.x; k < n4; k += stride) {
        float4 c = c4[k];
        if (MASK) {
            const uint32_t kp = kp4[k];
            c.x = (kp & 0xffu) ? c.x : f_inf();
            c.y = (kp & 0xff00u) ? c.y : f_inf();
            c.z = (kp & 0xff0000u) ? c.z : f_inf();
            c.w = (kp & 0xff000000u) ? c.w : f_inf();
        }
        float4 r;
        r.x = k_of(c.x, eps, s2);
        r.y = k_of(c.y, eps, s2);
        r.z = k_of(c.z, eps, s2);
        r.w = k_of(c.w, eps, s2);
        k4[k] = r;
    }
    for (int64_t k = n4 * 4 + (int64_t)blockIdx.x * kMapBlock + threadIdx.x; k < n; k += stride)
        K[k] = k_of((MASK && keep[k] == 0) ? f_inf() : C[k], eps, s2);
}

// log of a marginal (torch `a.log()`), n elements; sets `neg_flag` in
// stats[0] when an element is negative (the reference's `(a < 0).any()`).
// y64 (may be null): the same log in float64 of the float32 value, for the
// fused step's float64 potentials.
__global__ void __launch_bounds__(kMapBlock)
sk_log_marginal(const float *__restrict__ x, float *__restrict__ y, double *__restrict__ y64,
                int64_t n, uint32_t *__restrict__ stats, uint32_t neg_flag) {
    const int64_t k = (int64_t)blockIdx.x * kMapBlock + threadIdx.x;
    const float v = k < n ? x[k] : 0.f;
    if (k < n) {
        y[k] = logf(v);
        if (y64 != nullptr)
            y64[k] = log((double)v);
    }
    if (ballot(v < 0.f) != 0 && lane_id() == 0)
        atomicOr(&stats[0], neg_flag);
}

__global__ void __launch_bounds__(kMapBlock)
sk_fill(float *__restrict__ y, int64_t n, float value) {
    const int64_t k = (int64_t)blockIdx.x * kMapBlock + threadIdx.x;
    if (k < n)
        y[k] = value;
}

__global__ void __launch_bounds__(kMapBlock)
sk_fill64(double *__restrict__ y, int64_t n, double value) {
    const int64_t k = (int64_t)blockIdx.x * kMapBlock + threadIdx.x;
    if (k < n)
        y[k] = value;
}

// Start state of sk_prepare: every row and column flagged all-+inf, stats 0.
__global__ void __launch_bounds__(kMapBlock)
sk_reset_flags(uint8_t *__restrict__ inf_row, int64_t n_row, uint8_t *__restrict__ inf_col,
               int64_t n_col, uint32_t *__restrict__ stats) {
    const int64_t k = (int64_t)blockIdx.x * kMapBlock + threadIdx.x;
    if (k < n_row)
        inf_row[k] = 1;
    if (k < n_col)
        inf_col[k] = 1;
    if (k < 2)
        stats[k] = 0;
}

// One pass over the cost C (B, N, M) and the optional keep mask:
//   K         = -C'/e when e > 0 (as sk_log_kernel), C' = keep ? C : +inf
//   inf_row   cleared to 0 for each row of C' that holds a value other than
//             +inf (the reference's `(cost == inf).all(dim=2)`, negated)
//   inf_col   the same for columns
//   stats[0] |= kFlagNan / kFlagNegInf for NaN / -inf in C itself (the cost
//             is validated before the mask is fused into it)
//   stats[1]  = max(stats[1], order_key(largest finite C'))
// Block (x, y, z) covers the 64*CW columns from x*64*CW and `groups` groups
// of kPrepRows rows from y*groups*kPrepRows, of batch z.  Lanes own CW
// consecutive columns (4 with float4 loads, else 1); wave w reads rows
// w*8 .. w*8+7 of a group with all eight loads in flight (row indexes clamped
// to N-1, the surplus rows ignored).  A row flag is one byte store per wave;
// column flags are OR-ed over the waves in LDS and stored once per block; the
// stats words see at most one atomic each per block.  Flags are only ever
// cleared, so stores from different blocks cannot conflict.
template <bool VEC, bool MASK>
__global__ void __launch_bounds__(kPrepWaves * 64)
sk_prepare(const float *__restrict__ C, const uint8_t *__restrict__ keep,
           float *__restrict__ K, uint8_t *__restrict__ inf_row, uint8_t *__restrict__ inf_col,
           uint32_t *__restrict__ stats, int64_t N, int64_t M, int groups, float e, double s2) {
    constexpr int CW = VEC ? 4 : 1;
    __shared__ uint32_t col_any[kPrepWaves][64];
    __shared__ float blk_max[kPrepWaves];
    __shared__ uint32_t blk_flags[kPrepWaves];
    const int lane = lane_id();
    const int w = (int)(threadIdx.x >> 6);
    const int64_t b = blockIdx.z;
    const int64_t c0 = ((int64_t)blockIdx.x * 64 + lane) * CW;
    const bool col_ok = c0 < M;
    const int64_t cc = col_ok ? c0 : 0;  // column the loads use
    const bool write_k = e > 0.f;
    uint32_t any_col = 0;  // bit q: column c0 + q holds a C' value other than +inf
    bool nan = false, ninf = false;
    float vmax = -f_inf();
    for (int g = 0; g < groups; ++g) {
        const int64_t r0 =
            ((int64_t)blockIdx.y * groups + g) * kPrepRows + (int64_t)w * kPrepRowsPerWave;
        if (r0 >= N)
            break;
        float v[kPrepRowsPerWave][CW];
        uint32_t kp[kPrepRowsPerWave];
#pragma unroll
        for (int k = 0; k < kPrepRowsPerWave; ++k) {
            const int64_t r = r0 + k < N ? r0 + k : N - 1;
            const int64_t off = (b * N + r) * M + cc;
            if constexpr (VEC) {
                const float4 t = *reinterpret_cast<const float4 *>(C + off);
                v[k][0] = t.x;
                v[k][1] = t.y;
                v[k][2] = t.z;
                v[k][3] = t.w;
                kp[k] = MASK ? *reinterpret_cast<const uint32_t *>(keep + off) : ~0u;
            } else {
                v[k][0] = C[off];
                kp[k] = MASK ? (uint32_t)keep[off] : ~0u;
            }
        }
#pragma unroll
        for (int k = 0; k < kPrepRowsPerWave; ++k) {
            const int64_t r = r0 + k;
            if (r >= N)
                break;
            bool row_any = false;
            float kv[CW];
#pragma unroll
            for (int q = 0; q < CW; ++q) {
                const float x = col_ok ? v[k][q] : f_inf();
                nan = nan || x != x;
                ninf = ninf || x == -f_inf();
                const bool kept = !MASK || ((kp[k] >> (8 * q)) & 0xffu) != 0;
                const float y = kept ? x : f_inf();
                if (y != f_inf()) {
                    any_col |= 1u << q;
                    row_any = true;
                }
                if (__builtin_isfinite(y))
                    vmax = fmaxf(vmax, y);
                kv[q] = k_of(y, e, s2);
            }
            if (write_k && col_ok) {
                const int64_t off = (b * N + r) * M + c0;
                if constexpr (VEC)
                    *reinterpret_cast<float4 *>(K + off) = make_float4(kv[0], kv[1], kv[2], kv[3]);
                else
                    K[off] = kv[0];
            }
            if (ballot(row_any) != 0 && lane == 0)
                inf_row[b * N + r] = 0;
        }
    }
    const uint32_t fl = (ballot(nan) != 0 ? kFlagNan : 0u) | (ballot(ninf) != 0 ? kFlagNegInf : 0u);
    const float wm = wave_max(vmax);
    col_any[w][lane] = any_col;
    if (lane == 0) {
        blk_max[w] = wm;
        blk_flags[w] = fl;
    }
    __syncthreads();
    if (w != 0)
        return;
    uint32_t a = 0;
#pragma unroll
    for (int k = 0; k < kPrepWaves; ++k)
        a |= col_any[k][lane];
    if (col_ok && a != 0) {
        uint8_t *dst = inf_col + b * M + c0;
        if (VEC && a == 0xfu) {
            *reinterpret_cast<uint32_t *>(dst) = 0u;
        } else {
#pragma unroll
            for (int q = 0; q < CW; ++q)
                if ((a >> q) & 1u)
                    dst[q] = 0;
        }
    }
    if (lane == 0) {
        float m = blk_max[0];
        uint32_t f = blk_flags[0];
#pragma unroll
        for (int k = 1; k < kPrepWaves; ++k) {
            m = fmaxf(m, blk_max[k]);
            f |= blk_flags[k];
        }
        if (f != 0)
            atomicOr(&stats[0], f);
        if (m > -f_inf()) {
            const uint32_t key = order_key(m);
            if (key > __hip_atomic_load(&stats[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
                atomicMax(&stats[1], key);
        }
    }
}

// ---- row sweep: log_u -------------------------------------------------------------

__device__ __forceinline__ void row_lse_update(Lse acc, int64_t r, const float *__restrict__ log_mu,
                                               float *__restrict__ log_u, float damp,
                                               int unbalanced) {
    if (lane_id() == 0) {
        const float lse = lse_value(acc);
        log_u[r] = update_potential(lse, log_mu[r], log_u[r], damp, unbalanced != 0);
    }
}

// Each wave owns kRowsPerWave consecutive rows of one batch; M % 4 == 0 and
// M <= 256*kRowNV.  All the wave's row loads are issued before any reduction,
// and each row is an exact two-pass LSE over registers.
__global__ void __launch_bounds__(kRowWaves * 64)
sk_row_sweep(const float *__restrict__ K, const float *__restrict__ log_v,
             const float *__restrict__ log_mu, const uint8_t *__restrict__ inf_row,
             float *__restrict__ log_u, int64_t n_batch, int64_t N, int64_t M,
             int64_t waves_per_batch, float damp, int unbalanced) {
    const int64_t gw = (int64_t)blockIdx.x * kRowWaves + threadIdx.x / 64;
    const int64_t b = gw / waves_per_batch;
    if (b >= n_batch)
        return;  // surplus waves of the last block
    const int64_t i_begin = (gw % waves_per_batch) * kRowsPerWave;
    const int lane = lane_id();
    const int64_t m4 = M / 4;
    const float4 *lv4 = reinterpret_cast<const float4 *>(log_v + b * M);
    {  // m4 <= 64 * kRowNV here (longer rows take sk_row_sweep_split)
        float4 kk[kRowsPerWave][kRowNV];
#pragma unroll
        for (int rr = 0; rr < kRowsPerWave; ++rr) {
            const int64_t i = i_begin + rr;
            const float4 *row4 = reinterpret_cast<const float4 *>(K + (b * N + i) * M);
#pragma unroll
            for (int k = 0; k < kRowNV; ++k) {
                const int64_t q = (int64_t)k * 64 + lane;
                kk[rr][k] = (i < N && q < m4) ? row4[q]
                                              : make_float4(-f_inf(), -f_inf(), -f_inf(), -f_inf());
            }
        }
        float4 lv[kRowNV];
#pragma unroll
        for (int k = 0; k < kRowNV; ++k) {
            const int64_t q = (int64_t)k * 64 + lane;
            lv[k] = q < m4 ? lv4[q] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int rr = 0; rr < kRowsPerWave; ++rr) {
            const int64_t i = i_begin + rr;
            if (i >= N)
                break;
            const int64_t r = b * N + i;
            if (inf_row[r])
                continue;  // lse = -inf: log_u keeps its value
            float t[4 * kRowNV];
#pragma unroll
            for (int k = 0; k < kRowNV; ++k) {
                t[4 * k + 0] = kk[rr][k].x + lv[k].x;
                t[4 * k + 1] = kk[rr][k].y + lv[k].y;
                t[4 * k + 2] = kk[rr][k].z + lv[k].z;
                t[4 * k + 3] = kk[rr][k].w + lv[k].w;
            }
            float m = t[0];
#pragma unroll
            for (int k = 1; k < 4 * kRowNV; ++k)
                m = fmaxf(m, t[k]);
            m = wave_max_all(m);
            const float sh = lse_shift(m);
            float s = 0.f;
#pragma unroll
            for (int k = 0; k < 4 * kRowNV; ++k)
                s += exp_nonpos(t[k] - sh);
            s = wave_sum_all(s);
            row_lse_update(Lse{m, s}, r, log_mu, log_u, damp, unbalanced);
        }
    }
}

// Rows longer than one short-row chunk (M > 256*kRowNV, M % 4 == 0): a block
// of W waves owns one row; wave w takes chunks of 256*NV columns w, w+W, ...
// (each an exact two-pass LSE over registers, merged online when a wave has
// several), and the W partial (max, sum) pairs merge in LDS in wave order.
// Every wave keeps a whole chunk's loads in flight.  W = 8 with NV = 4
// (1024-column chunks, 50 VGPRs, eight waves per SIMD) measured best on C5:
// 351 us per iteration, against 365 with 2048-column chunks (82 VGPRs) and
// 376 with sixteen waves of one chunk each.
template <int W, int NV>
__global__ void __launch_bounds__(W * 64)
sk_row_sweep_split(const float *__restrict__ K, const float *__restrict__ log_v,
                   const float *__restrict__ log_mu, const uint8_t *__restrict__ inf_row,
                   float *__restrict__ log_u, int64_t N, int64_t M, float damp, int unbalanced) {
    const int64_t r = blockIdx.x;  // b * N + i
    if (inf_row[r])
        return;  // lse = -inf: log_u keeps its value
    const int64_t b = r / N;
    const int w = threadIdx.x / 64;
    const int lane = lane_id();
    const int64_t m4 = M / 4;
    constexpr int CH = 64 * NV;
    const float4 *row4 = reinterpret_cast<const float4 *>(K + r * M);
    const float4 *lv4 = reinterpret_cast<const float4 *>(log_v + b * M);
    Lse acc{-f_inf(), 0.f};
    for (int64_t base = (int64_t)w * CH; base < m4; base += (int64_t)W * CH) {
        float4 kk[NV], lv[NV];
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int64_t q = base + (int64_t)k * 64 + lane;
            kk[k] = q < m4 ? row4[q] : make_float4(-f_inf(), -f_inf(), -f_inf(), -f_inf());
        }
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int64_t q = base + (int64_t)k * 64 + lane;
            lv[k] = q < m4 ? lv4[q] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        float t[4 * NV];
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            t[4 * k + 0] = kk[k].x + lv[k].x;
            t[4 * k + 1] = kk[k].y + lv[k].y;
            t[4 * k + 2] = kk[k].z + lv[k].z;
            t[4 * k + 3] = kk[k].w + lv[k].w;
        }
        float m = t[0];
#pragma unroll
        for (int k = 1; k < 4 * NV; ++k)
            m = fmaxf(m, t[k]);
        m = wave_max_all(m);
        const float sh = lse_shift(m);
        float sum = 0.f;
#pragma unroll
        for (int k = 0; k < 4 * NV; ++k)
            sum += exp_nonpos(t[k] - sh);
        sum = wave_sum_all(sum);
        acc = lse_merge(acc, Lse{m, sum});
    }
    __shared__ float2 part[W];
    if (lane == 0)
        part[w] = make_float2(acc.m, acc.s);
    __syncthreads();
    if (threadIdx.x == 0) {
        Lse tot{part[0].x, part[0].y};
#pragma unroll
        for (int k = 1; k < W; ++k)
            tot = lse_merge(tot, Lse{part[k].x, part[k].y});
        log_u[r] = update_potential(lse_value(tot), log_mu[r], log_u[r], damp, unbalanced != 0);
    }
}

// Generic row sweep for M % 4 != 0: one wave per row, online LSE.
__global__ void __launch_bounds__(256)
sk_row_sweep_scalar(const float *__restrict__ K, const float *__restrict__ log_v,
                    const float *__restrict__ log_mu, const uint8_t *__restrict__ inf_row,
                    float *__restrict__ log_u, int64_t B, int64_t N, int64_t M, float damp,
                    int unbalanced) {
    const int64_t r = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
    if (r >= B * N)
        return;
    const int64_t b = r / N;
    const int lane = lane_id();
    if (inf_row[r])
        return;
    const float *row = K + r * M;
    const float *lv = log_v + b * M;
    Lse acc{-f_inf(), 0.f};
    for (int64_t j = lane; j < M; j += 64) {
        const float t = row[j] + lv[j];
        if (t > acc.m) {
            if (acc.s != 0.f)
                acc.s *= exp_nonpos(lse_shift(acc.m) - lse_shift(t));
            acc.m = t;
        }
        acc.s += exp_nonpos(t - lse_shift(acc.m));
    }
    acc = wave_lse(acc);
    if (lane == 0) {
        const float lse = lse_value(acc);
        log_u[r] = update_potential(lse, log_mu[r], log_u[r], damp, unbalanced != 0);
    }
}

// ---- column sweep: log_v ----------------------------------------------------------

// grid (n_strip, n_chunk, B), SW-column strips.  Thread tc = tid % (SW/4)
// owns columns strip*SW + 4*tc .. +3, row group tg = tid / (SW/4) folds rows
// chunk_start + tg, + G, ... (G = 256 / (SW/4) groups).  With one chunk the
// block finishes the LSE and updates log_v; otherwise it writes (max, sum)
// partials for sk_col_merge.
template <bool VEC, int SW>
__global__ void __launch_bounds__(kColThreads)
sk_col_sweep(const float *__restrict__ K, const float *__restrict__ log_u,
             const float *__restrict__ log_nu, const uint8_t *__restrict__ inf_col,
             float *__restrict__ log_v, float2 *__restrict__ colpart, int64_t N, int64_t M,
             int rows_per_chunk, int n_chunk, float damp, int unbalanced) {
    const int strip = blockIdx.x, chunk = blockIdx.y;
    const int64_t b = blockIdx.z;
    constexpr int G = kColThreads / (SW / 4);  // row groups
    const int tc = threadIdx.x % (SW / 4);
    const int tg = threadIdx.x / (SW / 4);
    const int64_t j0 = (int64_t)strip * SW + 4 * tc;
    const int64_t i0 = (int64_t)chunk * rows_per_chunk;
    const int64_t i1 = (i0 + rows_per_chunk < N) ? i0 + rows_per_chunk : N;
    const float *Kb = K + b * N * M;
    const float *lu = log_u + b * N;
    Lse acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
        acc[c] = Lse{-f_inf(), 0.f};
    const bool colok = j0 < M;
    for (int64_t ib = i0 + tg; ib < i1; ib += (int64_t)G * kColU) {
        float t[kColU][4];
#pragma unroll
        for (int u = 0; u < kColU; ++u) {
            const int64_t i = ib + (int64_t)u * G;
            if (colok && i < i1) {
                const float lui = lu[i];
                if (VEC) {
                    const float4 k4 = *reinterpret_cast<const float4 *>(Kb + i * M + j0);
                    t[u][0] = k4.x + lui;
                    t[u][1] = k4.y + lui;
                    t[u][2] = k4.z + lui;
                    t[u][3] = k4.w + lui;
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        t[u][c] = (j0 + c < M) ? Kb[i * M + j0 + c] + lui : -f_inf();
                }
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    t[u][c] = -f_inf();
            }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float gm = t[0][c];
#pragma unroll
            for (int u = 1; u < kColU; ++u)
                gm = fmaxf(gm, t[u][c]);
            if (gm > acc[c].m) {
                if (acc[c].s != 0.f)
                    acc[c].s *= exp_nonpos(lse_shift(acc[c].m) - lse_shift(gm));
                acc[c].m = gm;
            }
            const float sh = lse_shift(acc[c].m);
            float add = 0.f;
#pragma unroll
            for (int u = 0; u < kColU; ++u)
                add += exp_nonpos(t[u][c] - sh);
            acc[c].s += add;
        }
    }
    // merge the G row groups of each column in LDS
    __shared__ float2 part[G][SW];
#pragma unroll
    for (int c = 0; c < 4; ++c)
        part[tg][4 * tc + c] = make_float2(acc[c].m, acc[c].s);
    __syncthreads();
    if (threadIdx.x < SW) {
        const int cc = threadIdx.x;
        const int64_t j = (int64_t)strip * SW + cc;
        if (j < M) {
            Lse tot{-f_inf(), 0.f};
#pragma unroll
            for (int g = 0; g < G; ++g)
                tot = lse_merge(tot, Lse{part[g][cc].x, part[g][cc].y});
            if (n_chunk == 1) {
                const int64_t t = b * M + j;
                if (!inf_col[t]) {
                    const float lse = lse_value(tot);
                    log_v[t] = update_potential(lse, log_nu[t], log_v[t], damp, unbalanced != 0);
                }
            } else {
                colpart[(b * n_chunk + chunk) * M + j] = make_float2(tot.m, tot.s);
            }
        }
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

// ---- fused step: row sweep and column partials in one read of K ----------------------
//
// The column step of iteration s needs log_u of iteration s, which the row step
// produces one row at a time; the row is still in registers when its new log_u
// is known, so each row is folded into per-column sums right there.  One step
// then reads K once (B*N*M*4 bytes) instead of twice.  The column LSE of the
// step is the merge of the sums of every row chunk (sk_col_merge_blk),
// launched after the pass; the next step's row sweep needs that log_v, so the
// merge cannot move into the pass.
//
// Both LSEs work in base 2 on the native v_exp_f32, with K already in base-2
// units: y = K + p2 for the potential p2 scaled once (log_v per column in LDS,
// log_u per row).
//   row:    the sum of 2^(y - rs) against the row's LSE of the previous step
//           (a shift is only a scale: the sum keeps its relative precision
//           while it neither overflows nor underflows; accepted in [2^-16,
//           2^16]), else the exact two-pass (max, then sum of 2^(y - max)),
//           the reference's logsumexp;
//   column: the same terms times one per-row factor (fz_row), so a value costs
//           one add, one subtract, one exp and two fma in all.
// The first step, and the first after K changes, fold the columns with an
// exact running (max, sum) instead (EXACT instances).  v_exp_f32 issues at
// half the FMA rate.

constexpr float kFltMaxNeg = -3.402823466e38f;
constexpr float kShiftWindow = 16.f;  // accepted |LSE - shift|, base 2

// Clang vector (not HIP's float4 struct): arrays of it passed by reference to
// the inlined helpers below stay in registers.
typedef float vf4 __attribute__((ext_vector_type(4)));

// max without the NaN canonicalisation fmaxf costs on this target (two extra
// v_max per call): v_maximum3_f32.  The values here are never NaN (the cost
// is validated), and +-inf order as with fmaxf.
__device__ __forceinline__ float fmax_nn(float a, float b) {
    return __builtin_elementwise_maximum(a, b);
}

// base-2 log-sum-exp partial: m = max or shift of y (may be +-inf),
// s = sum 2^(y - shift(m))
__device__ __forceinline__ Lse lse2_merge(Lse p, Lse q) {
    const float m = fmaxf(p.m, q.m);
    const float sh = lse_shift(m);
    const float a = (p.s == 0.f) ? 0.f : p.s * __builtin_amdgcn_exp2f(lse_shift(p.m) - sh);
    const float c = (q.s == 0.f) ? 0.f : q.s * __builtin_amdgcn_exp2f(lse_shift(q.m) - sh);
    return Lse{m, a + c};
}

// base-2 LSE of a base-2 partial
__device__ __forceinline__ float lse2_log2(Lse p) { return __builtin_amdgcn_logf(p.s) + lse_shift(p.m); }

// exact running (max, sum) fold of one base-2 value: one exp per value,
// d = y - m;  e = 2^(-|d|);  s = d > 0 ? s*e + 1 : s + e;  m = max(m, y);
// m starts at -FLT_MAX rather than -inf so that y - m is never (-inf) - (-inf)
__device__ __forceinline__ void col_fold2(float &m, float &s, float y) {
    const float d = y - m;
    const float e = __builtin_amdgcn_exp2f(-fabsf(d));  // 0 for y = -inf
    s = d > 0.f ? fmaf(s, e, 1.f) : s + e;
    m = fmax_nn(m, y);
}

// (max, sum) of col_fold2 as a partial: a column that saw no value above -inf
// reads (-inf, 0), one that saw +inf reads (+inf, +inf), whose LSE is +inf as
// with torch's shift rule
__device__ __forceinline__ Lse fold_partial(float m, float s) {
    return Lse{s != 0.f ? m : -f_inf(), m == f_inf() ? f_inf() : s};
}

// Natural units per base-2 unit and back, float64: the fused step's K holds
// -C'*log2(e)/e (k_of with s2 = -kLog2eD/e) and its potentials enter the
// element loops scaled by kLog2eD, so 2^(K + p2) = e^(-C'/e + p) up to the
// float32 roundings of K and p2, with no constant's rounding in the exponent.
constexpr double kLog2eD = 1.4426950408889634074;
constexpr double kLn2D = 0.69314718055994530942;

// log2 of a float32 s > 0 in float64: s = m * 2^e with m in [sqrt(1/2),
// sqrt(2)), e exact and the native log on m only.  The native log is
// accurate near 1 but its error grows with |log2 s| (up to one float32 ulp
// of the result, biased low), and a bias common to every row or column is
// what the balanced potentials' neutral mode accumulates step after step.
// +inf, 0 and NaN go to the native log directly.
__device__ __forceinline__ double log2_split(float s) {
    if (!(s > 0.f) || !__builtin_isfinite(s))
        return (double)__builtin_amdgcn_logf(s);
    int e = __builtin_amdgcn_frexp_expf(s);
    float m = __builtin_amdgcn_frexp_mantf(s);  // [0.5, 1)
    if (m < 0.70710678f) {
        m *= 2.f;
        e -= 1;
    }
    return (double)e + (double)__builtin_amdgcn_logf(m);
}

// log2 of a float64 sum s > 0: log2_split of its float32 rounding plus the
// first-order term of the rounding (relative <= 2^-24, so the second-order
// term is below 2^-49).
__device__ __forceinline__ double log2_of_sum(double s) {
    const float h = (float)s;
    const float r = (float)(s - (double)h);  // exact: |r| <= ulp(h) / 2
    return log2_split(h) + (double)(r * __builtin_amdgcn_rcpf(h) * kLog2e);
}

// 2^t of a float64 t as a float32, to about 1e-7 relative: 2^round(t)
// exactly (ldexp) times the native 2^f of the float32 fraction f, |f| <= 1/2,
// with f's own rounding r restored to first order (2^(f + r) = 2^f (1 + r ln 2)).
__device__ __forceinline__ float pow2_of(double t) {
    const double ti = fmin(fmax(rint(t), -300.0), 300.0);
    const double fd = t - ti;
    const float f = (float)fd;
    const float r = (float)(fd - (double)f);
    const float e = __builtin_amdgcn_exp2f(f);
    return ldexpf(fmaf(e, r * kLn2, e), (int)ti);
}

// A potential p (float64) enters the float32 element loops as p2 = fl(p *
// log2 e) and the weight w = 2^(p * log2 e - p2) = 1 + (p*log2 e - p2) ln 2
// (to 1e-13), so a term 2^(K + p2) * w carries the potential's float64 value:
// the rounding of p2 is not a fixed error of every step's sums.
__device__ __forceinline__ float potential_weight(double p, float p2) {
    return (float)(1.0 + (p * kLog2eD - (double)p2) * kLn2D);
}

// The potential update in float64: the reference's isfinite keep-previous
// rule on the natural LSE l2 * ln 2, damping in float64 (the reference's
// rule and order, _log_sinkhorn.py:194-215, _unbalanced_sinkhorn.py:72-100).
__device__ __forceinline__ double update_potential64(double l2, double log_marg, double old,
                                                     double damp, bool unbalanced) {
    if (!isfinite(l2))
        return old;
    const double diff = log_marg - l2 * kLn2D;
    return unbalanced ? damp * diff : diff;
}

// All NV float4 of a row in flight at once: scalar row base + 32-bit lane
// byte offsets (the saddr form of the load).  Lanes past the row end read its
// last float4 again (offsets clamped); their log_v in LDS is -inf, which
// keeps them out of the row LSE, and their column sums are never stored.
// The row's float64 log marginal and potential and its previous base-2 LSE
// (its shift) are loaded with it: a load issued later would make the wait
// for it a wait for every row in flight.  A row of C' that is all +inf needs
// no flag: K is -inf on it, its terms are 0 and its sum 0 or NaN, which
// fails the window test; the exact LSE is then -inf and the potential keeps
// its value (the reference's keep-previous rule), and its column terms are 0.
// NT: non-temporal loads, for a K larger than the last-level (Infinity)
// cache, which each step streams once and would only evict what the next
// step reads (C5, 1 GiB: 187.9 against 193.7 us per step; C4's 256 MiB, which
// the cache partly keeps between steps, is faster with ordinary loads).
template <int NV, bool NT>
__device__ __forceinline__ void fz_load(vf4 (&dst)[NV], double &mu, double &u, float &rs,
                                        const vf4 *__restrict__ row4, const uint32_t (&qb)[NV],
                                        int64_t r, const double *__restrict__ mu64,
                                        const double *__restrict__ lu64,
                                        const float *__restrict__ lse2_row) {
    const char *base = reinterpret_cast<const char *>(row4);
    if constexpr (NT) {
#pragma unroll
        for (int k = 0; k < NV; ++k)
            dst[k] = __builtin_nontemporal_load(reinterpret_cast<const vf4 *>(base + qb[k]));
    } else {
#pragma unroll
        for (int k = 0; k < NV; ++k)
            dst[k] = *reinterpret_cast<const vf4 *>(base + qb[k]);
    }
    mu = mu64[r];
    u = lu64[r];
    rs = lse2_row[r];
}

// Exact base-2 LSE of one row (two passes over the row in registers: max,
// then sum of 2^(y - max)); the W waves of a row merge their (max, sum) pairs
// in LDS slot `par`.  Returns the slot parity for the next use.
template <int W, int NV>
__device__ __forceinline__ int fz_row_exact(const vf4 (&kk)[NV], const vf4 *lv_s,
                                            const vf4 (&wv)[NV], float2 (*rowpart)[W], int par,
                                            int w, int lane, Lse &tot) {
    float m = -f_inf();
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const vf4 y = kk[k] + lv_s[(k * W + w) * 64 + lane];
        m = fmax_nn(fmax_nn(m, y.x), y.y);
        m = fmax_nn(fmax_nn(m, y.z), y.w);
    }
    m = wave_max_all(m);
    const float sh = lse_shift(m);
    // y is formed again from log_v in LDS rather than kept in 32 VGPRs: the
    // pass is bound by the rows in flight per SIMD, and VGPRs buy rows
    asm volatile("" ::: "memory");
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const vf4 y = kk[k] + lv_s[(k * W + w) * 64 + lane];
        s = fmaf(__builtin_amdgcn_exp2f(y.x - sh), wv[k].x, s);
        s = fmaf(__builtin_amdgcn_exp2f(y.y - sh), wv[k].y, s);
        s = fmaf(__builtin_amdgcn_exp2f(y.z - sh), wv[k].z, s);
        s = fmaf(__builtin_amdgcn_exp2f(y.w - sh), wv[k].w, s);
    }
    s = (float)wave_sum_all_d((double)s);
    tot = Lse{m, s};
    if constexpr (W > 1) {
        if (lane == 0)
            rowpart[par][w] = make_float2(m, s);
        __syncthreads();
        tot = Lse{rowpart[par][0].x, rowpart[par][0].y};
#pragma unroll
        for (int k = 1; k < W; ++k)
            tot = lse2_merge(tot, Lse{rowpart[par][k].x, rowpart[par][k].y});
        par ^= 1;
    }
    return par;
}

// Outputs of the fused step's row update (row r): the float64 potential, its
// float32 copy (the caller's log_u), its kLog2eD-scaled float32 (what the
// column recompute adds) and the base-2 LSE (the next step's shift).
struct FzRowOut {
    double *lu64;
    float *log_u;
    float *lu2;
    float *lse2_row;
};

// The potential update and the column sums of a one-wave row (fz_row with
// W = 1, not EXACT) from its terms e_j = 2^(K_ij + lv2_j - shift).
template <int NV>
__device__ __forceinline__ void fz_row_tail_w1(const vf4 (&e)[NV], double l2, float shift,
                                               double mu_r, double u_r, int lane, int64_t r,
                                               const FzRowOut &out, double damp, int unbalanced,
                                               float (&cs)[4 * NV]) {
    const double lu = update_potential64(l2, mu_r, u_r, damp, unbalanced != 0);
    if (lane == 0) {
        out.lu64[r] = lu;
        out.log_u[r] = (float)lu;
        out.lu2[r] = (float)(lu * kLog2eD);
        out.lse2_row[r] = (float)l2;
    }
    const float a = pow2_of(lu * kLog2eD + (double)shift);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        cs[4 * k + 0] = fmaf(e[k].x, a, cs[4 * k + 0]);
        cs[4 * k + 1] = fmaf(e[k].y, a, cs[4 * k + 1]);
        cs[4 * k + 2] = fmaf(e[k].z, a, cs[4 * k + 2]);
        cs[4 * k + 3] = fmaf(e[k].w, a, cs[4 * k + 3]);
    }
}

// One row (batch-flat index r) of the fused step: its base-2 LSE, the log_u
// update in float64, then the row's share of the column sums.
//
// Row LSE: the terms e_j = 2^(K_ij + lv2_j - rs), weighted by the lv2
// rounding weights, summed against the row's LSE of the previous step (rs)
// in one pass and accepted when the sum lies in [sum_lo, sum_hi]; otherwise
// the row is read again and takes the exact two-pass (fz_row_exact), and the
// terms are formed again against its shift.
//
// Column sums (not EXACT): the column half-step needs 2^(K_ij + lu2_i - c)
// for the new log_u of this row.  That term is e_j * A_i * 2^(-lv2_j - c)
// with A_i = 2^(lu_i * log2 e + shift_i): the row's terms times one
// per-row factor, the last factor per column only.  So the row adds
// e_j * A_i to column j's sum (one fma per term, the terms already in
// registers), and the merge takes LSE2_j = log2(T_j) - lv2_j of the total
// T_j, the column's own factor folded in exactly.  A_i carries the float64
// potential (pow2_of), so no rounding of lu2 enters the columns.
//
// EXACT steps (the first, and the first after an epsilon change) fold the
// columns with a running (max, sum) instead (col_fold2), from y = K + lu2.
// Returns the LDS slot parity for the next row.
template <int W, int NV, bool EXACT>
__device__ __forceinline__ int fz_row(vf4 (&kk)[NV], double mu_r, double u_r, float rs,
                                      const vf4 *row4, const uint32_t (&qb)[NV],
                                      const vf4 *lv_s, const vf4 (&wv)[NV],
                                      float2 (*rowpart)[W], double (*rowsum)[W], int par, int w,
                                      int lane, int64_t r, const FzRowOut &out, float sum_lo,
                                      float sum_hi, double damp, int unbalanced,
                                      float (&cm)[EXACT ? 4 * NV : 1], float (&cs)[4 * NV]) {
    // u_r and rs were read with the row, before the row barrier after which
    // the row's potential and shift are rewritten
    double l2 = 0.0;
    float shift = rs;
    bool have = false;
    if constexpr (!EXACT) {
        // the terms replace the row's K in registers; lane sums in float32,
        // the wave's and the row's sums in float64 (wave_sum_all_d)
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const vf4 y = kk[k] + lv_s[(k * W + w) * 64 + lane];
            const vf4 e = vf4{__builtin_amdgcn_exp2f(y.x - rs), __builtin_amdgcn_exp2f(y.y - rs),
                              __builtin_amdgcn_exp2f(y.z - rs), __builtin_amdgcn_exp2f(y.w - rs)};
            kk[k] = e;
            s = fmaf(e.x, wv[k].x, s);
            s = fmaf(e.y, wv[k].y, s);
            s = fmaf(e.z, wv[k].z, s);
            s = fmaf(e.w, wv[k].w, s);
        }
        double s64 = wave_sum_all_d((double)s);
        if constexpr (W == 1) {
            // A one-wave row gives the rare exact fallback a tail and row
            // registers of its own.  When the fallback reloaded the row into
            // the registers of the common path, the compiler had the common
            // path wait for that (conditional) reload, and with it for the
            // next row's loads already in flight, on every row (C4: 38.3 ->
            // 37.4 us per iteration without that wait).  Rows split over
            // waves keep the form below: rewritten like this, the 16-wave
            // shape measured 2-3% slower.
            if (s64 >= (double)sum_lo && s64 <= (double)sum_hi) {  // false for NaN
                fz_row_tail_w1<NV>(kk, log2_of_sum(s64) + (double)rs, rs, mu_r, u_r, lane, r, out,
                                   damp, unbalanced, cs);
                return par;
            }
            vf4 kx[NV];
            const char *base = reinterpret_cast<const char *>(row4);
#pragma unroll
            for (int k = 0; k < NV; ++k)
                kx[k] = *reinterpret_cast<const vf4 *>(base + qb[k]);
            Lse tot;
            par = fz_row_exact<W, NV>(kx, lv_s, wv, rowpart, par, w, lane, tot);
            const float sh = lse_shift(tot.m);
#pragma unroll
            for (int k = 0; k < NV; ++k) {
                const vf4 y = kx[k] + lv_s[(k * W + w) * 64 + lane];
                kx[k] = vf4{__builtin_amdgcn_exp2f(y.x - sh), __builtin_amdgcn_exp2f(y.y - sh),
                            __builtin_amdgcn_exp2f(y.z - sh), __builtin_amdgcn_exp2f(y.w - sh)};
            }
            fz_row_tail_w1<NV>(kx, log2_split(tot.s) + (double)sh, sh, mu_r, u_r, lane, r, out,
                               damp, unbalanced, cs);
            return par;
        }
        if constexpr (W > 1) {  // the W waves' sums, added in LDS in wave order
            if (lane == 0)
                rowsum[par][w] = s64;
            __syncthreads();
            s64 = rowsum[par][0];
#pragma unroll
            for (int k = 1; k < W; ++k)
                s64 += rowsum[par][k];
            par ^= 1;
        }
        if (s64 >= (double)sum_lo && s64 <= (double)sum_hi) {  // block-uniform; false for NaN
            l2 = log2_of_sum(s64) + (double)rs;
            have = true;
        } else {
            // the exact two-pass needs the row's K again (rare: a stale shift)
            const char *base = reinterpret_cast<const char *>(row4);
#pragma unroll
            for (int k = 0; k < NV; ++k)
                kk[k] = *reinterpret_cast<const vf4 *>(base + qb[k]);
        }
    }
    if (!have) {
        Lse tot;
        par = fz_row_exact<W, NV>(kk, lv_s, wv, rowpart, par, w, lane, tot);
        shift = lse_shift(tot.m);
        l2 = log2_split(tot.s) + (double)shift;
        if constexpr (!EXACT) {
#pragma unroll
            for (int k = 0; k < NV; ++k) {
                const vf4 y = kk[k] + lv_s[(k * W + w) * 64 + lane];
                kk[k] = vf4{__builtin_amdgcn_exp2f(y.x - shift), __builtin_amdgcn_exp2f(y.y - shift),
                            __builtin_amdgcn_exp2f(y.z - shift), __builtin_amdgcn_exp2f(y.w - shift)};
            }
        }
    }
    // the update in float64: nothing of the potential is rounded to float32
    // between steps
    const double lu = update_potential64(l2, mu_r, u_r, damp, unbalanced != 0);
    const float lu2 = (float)(lu * kLog2eD);
    if (w == 0 && lane == 0) {
        out.lu64[r] = lu;
        out.log_u[r] = (float)lu;
        out.lu2[r] = lu2;
        out.lse2_row[r] = (float)l2;
    }
    if constexpr (EXACT) {
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const vf4 y = kk[k] + lu2;
            col_fold2(cm[4 * k + 0], cs[4 * k + 0], y.x);
            col_fold2(cm[4 * k + 1], cs[4 * k + 1], y.y);
            col_fold2(cm[4 * k + 2], cs[4 * k + 2], y.z);
            col_fold2(cm[4 * k + 3], cs[4 * k + 3], y.w);
        }
    } else {
        const float a = pow2_of(lu * kLog2eD + (double)shift);
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            cs[4 * k + 0] = fmaf(kk[k].x, a, cs[4 * k + 0]);
            cs[4 * k + 1] = fmaf(kk[k].y, a, cs[4 * k + 1]);
            cs[4 * k + 2] = fmaf(kk[k].z, a, cs[4 * k + 2]);
            cs[4 * k + 3] = fmaf(kk[k].w, a, cs[4 * k + 3]);
        }
    }
    return par;
}

// grid (n_chunk, B), block W*RW waves.  Chunk c of batch b holds the rows
// [c*rows_per_chunk, (c+1)*rows_per_chunk) or, interleaved, the rows c,
// c + n_chunk, c + 2*n_chunk, ... (the blocks of a batch then march through
// its rows side by side).  A row spans W waves: wave (g, w) of row group g
// owns float4 columns q = (k*W + w)*64 + lane, k < NV, of the chunk's rows
// number g, g + RW, ...  The first rows' loads go out before the block fills
// LDS, so they overlap that prologue.  With W > 1 the W (max, sum)
// pairs of a row merge in LDS (one barrier per row, double-buffered slots;
// RW = 1 then, so every wave of the block sees the same rows and the same
// barriers).  With RW > 1 the row groups' column sums add up in LDS after the
// last row.  NB: row buffers per wave.  colpart receives one float per column
// (the chunk's share of T_j = sum_i e_ij * A_i, fz_row), or with EXACT the
// exact running (max, sum) pair of col_fold2 (the first step, and the first
// after an epsilon change, have no usable row shift).  K holds the base-2 log
// kernel -C'*log2(e)/e and lv2 the kLog2eD-scaled log_v.  Requires M % 4 == 0,
// M <= 256*W*NV, 16-byte aligned K and lv2.
template <int W, int RW, int NV, int NB, bool EXACT, bool NT>
__global__ void __launch_bounds__(W * RW * 64)
sk_fused_step(const float *__restrict__ K, const float *__restrict__ lv2,
              const float *__restrict__ lvw, float *__restrict__ lse2_row,
              const double *__restrict__ mu64, double *__restrict__ lu64, float *__restrict__ log_u, float *__restrict__ lu2,
              float2 *__restrict__ colpart, int64_t N, int64_t M, int n_chunk,
              int rows_per_chunk, int interleave, float sum_lo, float sum_hi, double damp,
              int unbalanced) {
    static_assert(W == 1 || RW == 1, "a row is split over waves only with one row group");
    constexpr int MV = W * 64 * NV;  // float4 per row at most
    __shared__ vf4 lv_s[MV];         // log_v * log2(e) of the batch, -inf past M
    __shared__ float2 rowpart[2][W];
    __shared__ double rowsum[2][W];
    const int chunk = blockIdx.x;
    const int64_t b = blockIdx.y;
    // wave-uniform (readfirstlane): row addresses and loop bounds stay scalar
    const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int w = wid % W, g = wid / W;
    const int lane = lane_id();
    const int64_t m4 = M / 4;
    // this wave's rows: i = first, first + step, ... < end
    const int64_t first = interleave ? chunk + (int64_t)n_chunk * g
                                     : (int64_t)chunk * rows_per_chunk + g;
    const int64_t step = interleave ? (int64_t)n_chunk * RW : RW;
    const int64_t end = interleave ? N
                        : ((int64_t)(chunk + 1) * rows_per_chunk < N
                               ? (int64_t)(chunk + 1) * rows_per_chunk
                               : N);

    uint32_t qb[NV];  // byte offset of the lane's float4 k in a row (clamped)
    bool qok[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int q = (k * W + w) * 64 + lane;
        qok[k] = q < m4;
        qb[k] = 16u * (uint32_t)(qok[k] ? q : (int)m4 - 1);
    }
    // the lane's columns' weights (potential_weight of log_v): lane-private,
    // so held in registers for the whole pass
    vf4 wv[NV];
    {
        const vf4 *w4 = reinterpret_cast<const vf4 *>(lvw + b * M);
#pragma unroll
        for (int k = 0; k < NV; ++k)
            wv[k] = qok[k] ? w4[(k * W + w) * 64 + lane] : vf4{1.f, 1.f, 1.f, 1.f};
    }
    float cs[4 * NV], cm[EXACT ? 4 * NV : 1];
#pragma unroll
    for (int k = 0; k < 4 * NV; ++k)
        cs[k] = 0.f;
#pragma unroll
    for (int k = 0; k < (EXACT ? 4 * NV : 1); ++k)
        cm[k] = kFltMaxNeg;
    const vf4 *Kb4 = reinterpret_cast<const vf4 *>(K + b * N * M);
    const int64_t rb = b * N;
    const FzRowOut out{lu64, log_u, lu2, lse2_row};
    int par = 0;
    int64_t i = first;
    // NB row buffers: a wave keeps NB - 1 rows' loads in flight while it
    // reduces one (NB = 1: the next row's loads go out once a row is folded)
    vf4 kr[NB][NV];
    double rmu[NB], ru[NB];
    float rls[NB];
#define TM_FZ_LOAD(P_, I_)                                                                    \
    fz_load<NV, NT>(kr[P_], rmu[P_], ru[P_], rls[P_], Kb4 + (I_) * m4, qb, rb + (I_), mu64, \
                    lu64, lse2_row)
    // the wave's last row; prefetches past it load it again, so that every
    // path through the loop issues the same loads and the wait for a row's
    // data can leave the rows prefetched after it in flight (a conditional
    // prefetch makes the compiler wait for every outstanding load instead)
    const int64_t last = i < end ? first + ((end - 1 - first) / step) * step : first;
    if constexpr (NB == 1) {
        if (i < end)
            TM_FZ_LOAD(0, i);
    } else {
        if (i < end) {
#pragma unroll
            for (int p = 0; p < NB - 1; ++p)
                TM_FZ_LOAD(p, i + p * step <= last ? i + p * step : last);
        }
    }
    const float4 *lv4 = reinterpret_cast<const float4 *>(lv2 + b * M);
    for (int q = threadIdx.x; q < MV; q += W * RW * 64) {
        const float4 v = q < m4 ? lv4[q] : make_float4(-f_inf(), -f_inf(), -f_inf(), -f_inf());
        lv_s[q] = vf4{v.x, v.y, v.z, v.w};
    }
    __syncthreads();

    if constexpr (NB == 1) {
        for (; i < end; i += step) {
            par = fz_row<W, NV, EXACT>(kr[0], rmu[0], ru[0], rls[0], Kb4 + i * m4, qb, lv_s, wv,
                                       rowpart, rowsum, par, w, lane, rb + i, out, sum_lo, sum_hi,
                                       damp, unbalanced, cm, cs);
            if (i + step < end)
                TM_FZ_LOAD(0, i + step);
        }
    } else {
        while (i < end) {
#pragma unroll
            for (int p = 0; p < NB; ++p) {
                const int64_t ia = i + (int64_t)(NB - 1) * step;
                TM_FZ_LOAD((p + NB - 1) % NB, ia <= last ? ia : last);
                par = fz_row<W, NV, EXACT>(kr[p], rmu[p], ru[p], rls[p], Kb4 + i * m4, qb, lv_s,
                                           wv, rowpart, rowsum, par, w, lane, rb + i, out,
                                           sum_lo, sum_hi, damp, unbalanced, cm, cs);
                i += step;
                if (i >= end)
                    break;
            }
        }
    }
#undef TM_FZ_LOAD

    // add the row groups' sums (same columns, same shifts) in LDS: g >= h/2
    // hands over to g - h/2, halving until row group 0 holds the chunk's sum
    if constexpr (RW > 1) {
        __shared__ vf4 xs[RW / 2][NV][64];
        __shared__ vf4 xm[EXACT ? RW / 2 : 1][NV][64];
        for (int h = RW; h > 1; h >>= 1) {
            const int half = h >> 1;
            if (g >= half && g < h) {
#pragma unroll
                for (int k = 0; k < NV; ++k) {
                    xs[g - half][k][lane] = vf4{cs[4 * k], cs[4 * k + 1], cs[4 * k + 2],
                                                cs[4 * k + 3]};
                    if constexpr (EXACT)
                        xm[g - half][k][lane] = vf4{cm[4 * k], cm[4 * k + 1], cm[4 * k + 2],
                                                    cm[4 * k + 3]};
                }
            }
            __syncthreads();
            if (g < half) {
#pragma unroll
                for (int k = 0; k < NV; ++k) {
                    const vf4 o = xs[g][k][lane];
                    if constexpr (EXACT) {
                        const vf4 om = xm[g][k][lane];
                        const float pm[4] = {om.x, om.y, om.z, om.w};
                        const float ps[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            const Lse mrg = lse2_merge(fold_partial(cm[4 * k + c], cs[4 * k + c]),
                                                       fold_partial(pm[c], ps[c]));
                            cm[4 * k + c] = mrg.s != 0.f ? mrg.m : kFltMaxNeg;
                            cs[4 * k + c] = mrg.s;
                        }
                    } else {
                        cs[4 * k + 0] += o.x;
                        cs[4 * k + 1] += o.y;
                        cs[4 * k + 2] += o.z;
                        cs[4 * k + 3] += o.w;
                    }
                }
            }
            __syncthreads();
        }
    }
    if (g != 0)
        return;
    float2 *dst = colpart + (b * n_chunk + chunk) * M;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        if (qok[k]) {
            if constexpr (EXACT) {
                float4 *d4 = reinterpret_cast<float4 *>(dst + qb[k] / 4);
                Lse p[4];
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    p[c] = fold_partial(cm[4 * k + c], cs[4 * k + c]);
                d4[0] = make_float4(p[0].m, p[0].s, p[1].m, p[1].s);
                d4[1] = make_float4(p[2].m, p[2].s, p[3].m, p[3].s);
            } else {
                // the chunk's share of T_j alone (the float view of the same
                // buffer, chunk-major)
                float *sum = reinterpret_cast<float *>(colpart) + (b * n_chunk + chunk) * M;
                *reinterpret_cast<float4 *>(sum + qb[k] / 4) =
                    make_float4(cs[4 * k + 0], cs[4 * k + 1], cs[4 * k + 2], cs[4 * k + 3]);
            }
        }
    }
}

// Outputs of the merge's column update (column t): the float64 potential,
// its float32 copy (the caller's log_v), its kLog2eD-scaled float32 (the next
// pass's lv2) and the base-2 LSE (the next step's shift).
struct MergeOut {
    double *lv64;
    float *log_v;
    float *lv2;  // read (the pass's lv2) before it is rewritten
    float *lvw;  // potential_weight of the column's lv2
};

// grid (ceil(M/64), B), MW waves (16 for many chunks, else 4): lanes are 64
// consecutive columns (coalesced 512-byte reads of one chunk), wave w merges
// the partials of chunks w, w+MW, ..., and the waves merge in LDS.  Plain
// partials (exact = 0) are the chunks' shares of T_j (fz_row), added in
// float64; the column's base-2 LSE is log2(T_j) - lv2_j with the lv2 the pass
// used.  A column whose T_j lies outside [col_lo, col_hi] = [2^-96, 2^96]
// (its terms near float32 underflow or overflow) is recomputed exactly: the
// block then folds its 64 columns of every row of K with the step's lu2
// (wave w takes rows w, w+MW, ...).  Wave 0 updates the column's potential
// in float64.
template <int kMergeWaves>
__global__ void __launch_bounds__(kMergeWaves * 64)
sk_col_merge_blk(const float2 *__restrict__ colpart, const float *__restrict__ K,
                 const float *__restrict__ lu2, const double *__restrict__ nu64,
                 const uint8_t *__restrict__ inf_col, MergeOut out, int64_t N, int64_t M,
                 int n_chunk, int exact, double col_lo, double col_hi, double damp,
                 int unbalanced) {
    const int64_t b = blockIdx.y;
    const int w = (int)(threadIdx.x >> 6);
    const int lane = lane_id();
    const int64_t j = (int64_t)blockIdx.x * 64 + lane;
    const int64_t jj = j < M ? j : M - 1;
    const int64_t t = b * M + jj;
    // the column's own values are loaded before the partials, so that their
    // latency overlaps the partials' instead of following the LDS merge
    const double nu_t = nu64[t], v_t = out.lv64[t];
    const float lv2_t = out.lv2[t];
    const bool live = j < M && !inf_col[t];
    __shared__ float2 part[kMergeWaves][64];
    __shared__ double part64[kMergeWaves][64];
    int c = w;
    double l2;
    bool ok = true;
    if (exact) {  // (max, sum) pairs
        Lse acc{-f_inf(), 0.f};
        for (; c + 3 * kMergeWaves < n_chunk; c += 4 * kMergeWaves) {
            float2 p[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                p[u] = colpart[(b * n_chunk + c + u * kMergeWaves) * M + jj];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                acc = lse2_merge(acc, Lse{p[u].x, p[u].y});
        }
        for (; c < n_chunk; c += kMergeWaves) {
            const float2 p = colpart[(b * n_chunk + c) * M + jj];
            acc = lse2_merge(acc, Lse{p.x, p.y});
        }
        part[w][lane] = make_float2(acc.m, acc.s);
        __syncthreads();
#pragma unroll
        for (int k = 0; k < kMergeWaves; ++k)
            if (k != w)
                acc = lse2_merge(acc, Lse{part[k][lane].x, part[k][lane].y});
        l2 = log2_split(acc.s) + (double)lse_shift(acc.m);
    } else {  // shares of T_j: plain adds, in float64
        const float *sum = reinterpret_cast<const float *>(colpart);
        double tsum = 0.0;
        // sixteen loads in flight, then the same adds in the same order as
        // the four-load loop below
        for (; c + 15 * kMergeWaves < n_chunk; c += 16 * kMergeWaves) {
            float p[16];
#pragma unroll
            for (int u = 0; u < 16; ++u)
                p[u] = sum[(b * n_chunk + c + u * kMergeWaves) * M + jj];
#pragma unroll
            for (int q = 0; q < 16; q += 4)
                tsum += ((double)p[q] + (double)p[q + 1]) + ((double)p[q + 2] + (double)p[q + 3]);
        }
        for (; c + 7 * kMergeWaves < n_chunk; c += 8 * kMergeWaves) {
            float p[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                p[u] = sum[(b * n_chunk + c + u * kMergeWaves) * M + jj];
#pragma unroll
            for (int q = 0; q < 8; q += 4)
                tsum += ((double)p[q] + (double)p[q + 1]) + ((double)p[q + 2] + (double)p[q + 3]);
        }
        for (; c + 3 * kMergeWaves < n_chunk; c += 4 * kMergeWaves) {
            float p[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                p[u] = sum[(b * n_chunk + c + u * kMergeWaves) * M + jj];
            tsum += ((double)p[0] + (double)p[1]) + ((double)p[2] + (double)p[3]);
        }
        for (; c < n_chunk; c += kMergeWaves)
            tsum += (double)sum[(b * n_chunk + c) * M + jj];
        part64[w][lane] = tsum;
        __syncthreads();
        tsum = part64[0][lane];
#pragma unroll
        for (int k = 1; k < kMergeWaves; ++k)
            tsum += part64[k][lane];
        ok = tsum >= col_lo && tsum <= col_hi;  // false for NaN
        l2 = ok ? log2_of_sum(tsum) - (double)lv2_t : 0.0;
    }
    if (__syncthreads_or(live && !ok)) {
        float m = kFltMaxNeg, s = 0.f;
        const float *col = K + b * N * M + jj;
        for (int64_t i = w; i < N; i += kMergeWaves)
            col_fold2(m, s, col[i * M] + lu2[b * N + i]);
        part[w][lane] = make_float2(m, s);
        __syncthreads();
        Lse ex = fold_partial(part[0][lane].x, part[0][lane].y);
#pragma unroll
        for (int k = 1; k < kMergeWaves; ++k)
            ex = lse2_merge(ex, fold_partial(part[k][lane].x, part[k][lane].y));
        if (!ok)
            l2 = log2_split(ex.s) + (double)lse_shift(ex.m);
    }
    if (w != 0 || !live)
        return;
    const double lv = update_potential64(l2, nu_t, v_t, damp, unbalanced != 0);
    const float lv2 = (float)(lv * kLog2eD);
    out.lv64[t] = lv;
    out.log_v[t] = (float)lv;
    out.lv2[t] = lv2;
    out.lvw[t] = potential_weight(lv, lv2);
}

// ---- final plan -------------------------------------------------------------------

// log_plan[b,i,j] = (log_u[b,i] + K[b,i,j]) + log_v[b,j], K holding -C'/e_final
// from the last step (the reference's `(log_u + (-cost / eps)) + log_v`, the
// same float32 division); float4 rows when M % 4 == 0, generic otherwise.
__global__ void __launch_bounds__(kMapBlock)
sk_plan4(const float *__restrict__ K, const float *__restrict__ log_u,
         const float *__restrict__ log_v, float *__restrict__ plan, int64_t B, int64_t N,
         int64_t M) {
    const int64_t m4 = M / 4;
    const int64_t n4 = B * N * m4;
    const int64_t stride = (int64_t)gridDim.x * kMapBlock;
    const float4 *k4 = reinterpret_cast<const float4 *>(K);
    float4 *p4 = reinterpret_cast<float4 *>(plan);
    for (int64_t k = (int64_t)blockIdx.x * kMapBlock + threadIdx.x; k < n4; k += stride) {
        const int64_t row = k / m4;
        const int64_t q = k - row * m4;
        const int64_t b = row / N;
        const float u = log_u[row];
        const float4 v = reinterpret_cast<const float4 *>(log_v + b * M)[q];
        const float4 c = k4[k];
        float4 o;
        o.x = (u + c.x) + v.x;
        o.y = (u + c.y) + v.y;
        o.z = (u + c.z) + v.z;
        o.w = (u + c.w) + v.w;
        p4[k] = o;
    }
}

__global__ void __launch_bounds__(kMapBlock)
sk_plan(const float *__restrict__ K, const float *__restrict__ log_u,
        const float *__restrict__ log_v, float *__restrict__ plan, int64_t B, int64_t N,
        int64_t M) {
    const int64_t n = B * N * M;
    const int64_t stride = (int64_t)gridDim.x * kMapBlock;
    for (int64_t k = (int64_t)blockIdx.x * kMapBlock + threadIdx.x; k < n; k += stride) {
        const int64_t row = k / M;
        const int64_t j = k - row * M;
        const int64_t b = row / N;
        plan[k] = (log_u[row] + K[k]) + log_v[b * M + j];
    }
}

// The fused step's plan: log_plan[b,i,j] = lu64[b,i] + Kref[b,i,j] + lv64[b,j]
// in float64, rounded once, with Kref = -C'/e_final the reference's float32
// K (IEEE division; C' = +inf where the keep mask is false).  Float4 steps
// when `vec` (M % 4 == 0; C, plan 16-byte and keep 4-byte aligned).
template <bool MASK>
__global__ void __launch_bounds__(kMapBlock)
sk_plan64(const float *__restrict__ C, const uint8_t *__restrict__ keep,
          const double *__restrict__ lu64, const double *__restrict__ lv64,
          float *__restrict__ plan, int64_t B, int64_t N, int64_t M, float e, int vec) {
    const int64_t stride = (int64_t)gridDim.x * kMapBlock;
    if (vec) {
        const int64_t m4 = M / 4;
        const int64_t n4 = B * N * m4;
        const float4 *c4 = reinterpret_cast<const float4 *>(C);
        const uint32_t *kp4 = reinterpret_cast<const uint32_t *>(keep);
        float4 *p4 = reinterpret_cast<float4 *>(plan);
        for (int64_t k = (int64_t)blockIdx.x * kMapBlock + threadIdx.x; k < n4; k += stride) {
            const int64_t row = k / m4;
            const int64_t q = k - row * m4;
            const int64_t b = row / N;
            const double u = lu64[row];
            const double *v = lv64 + b * M + 4 * q;
            float4 c = c4[k];
            if (MASK) {
                const uint32_t kp = kp4[k];
                c.x = (kp & 0xffu) ? c.x : f_inf();
                c.y = (kp & 0xff00u) ? c.y : f_inf();
                c.z = (kp & 0xff0000u) ? c.z : f_inf();
                c.w = (kp & 0xff000000u) ? c.w : f_inf();
            }
            float4 o;
            o.x = (float)((u + (double)(-c.x / e)) + v[0]);
            o.y = (float)((u + (double)(-c.y / e)) + v[1]);
            o.z = (float)((u + (double)(-c.z / e)) + v[2]);
            o.w = (float)((u + (double)(-c.w / e)) + v[3]);
            p4[k] = o;
        }
        return;
    }
    const int64_t n = B * N * M;
    for (int64_t k = (int64_t)blockIdx.x * kMapBlock + threadIdx.x; k < n; k += stride) {
        const int64_t row = k / M;
        const int64_t j = k - row * M;
        const int64_t b = row / N;
        const float c = (MASK && keep[k] == 0) ? f_inf() : C[k];
        plan[k] = (float)((lu64[row] + (double)(-c / e)) + lv64[b * M + j]);
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

namespace {

#define TM_LAUNCH(...)                                                                    \
    do {                                                                                  \
        hipLaunchKernelGGL(__VA_ARGS__);                                                  \
        if (hipGetLastError() != hipSuccess)                                              \
            return TM_ERR_LAUNCH;                                                         \
    } while (0)

// Shape limits of the launch grids below.  Launches that put the batch on
// a grid dimension run in slices of at most kBatchSlice problems (pointers
// offset to the slice), so the batch size itself has no grid limit.
constexpr int64_t kBatchSlice = 65535;
bool shape_supported(const SinkhornLayout &L) {
    return L.n_strip <= 0x7fffffff && L.n_chunk <= 65535 && L.B * L.N <= 0x7fffffff;
}

// K for one epsilon: the reference's -C'/e (two-sweep step), or with `base2`
// the fused step's -C'*log2(e)/e.
int launch_log_kernel(const float *cost, const uint8_t *keep, float *K, int64_t nK, float e,
                      bool base2, hipStream_t stream) {
    const double s2 = base2 ? -kLog2eD / (double)e : 0.0;
    const int vec = ((uintptr_t)cost % 16) == 0 && ((uintptr_t)K % 16) == 0 &&
                    ((uintptr_t)keep % 4) == 0;
    const dim3 grid(grid_for(nK / 4 + 1, kMapBlock, 8192));
    if (keep != nullptr)
        TM_LAUNCH(sk_log_kernel<true>, grid, dim3(kMapBlock), 0, stream, cost, keep, K, nK, e,
                  s2, vec);
    else
        TM_LAUNCH(sk_log_kernel<false>, grid, dim3(kMapBlock), 0, stream, cost, keep, K, nK, e,
                  s2, vec);
    return TM_OK;
}

// The two-sweep column sweep, batch slices on grid z.
int launch_col_sweep(const SinkhornLayout &L, bool vec, const float *K, const float *log_u,
                     const float *log_nu, const uint8_t *inf_col, float *log_v, float2 *colpart,
                     float damp, int ub, hipStream_t stream) {
    const int64_t N = L.N, M = L.M;
    for (int64_t b0 = 0; b0 < L.B; b0 += kBatchSlice) {
        const int64_t nb = L.B - b0 < kBatchSlice ? L.B - b0 : kBatchSlice;
        const dim3 grid((unsigned)L.n_strip, (unsigned)L.n_chunk, (unsigned)nb);
        const float *k = K + b0 * N * M;
        const float *lu = log_u + b0 * N;
        const float *ln = log_nu + b0 * M;
        const uint8_t *ic = inf_col + b0 * M;
        float *lv = log_v + b0 * M;
        float2 *cp = colpart + b0 * L.n_chunk * M;
#define TM_COL_SWEEP(V_, S_)                                                                  \
    TM_LAUNCH((sk_col_sweep<V_, S_>), grid, dim3(kColThreads), 0, stream, k, lu, ln, ic, lv, cp, \
              N, M, L.rows_per_chunk, L.n_chunk, damp, ub)
        if (vec && L.strip == kColStripNarrow)
            TM_COL_SWEEP(true, kColStripNarrow);
        else if (vec)
            TM_COL_SWEEP(true, kColStrip);
        else if (L.strip == kColStripNarrow)
            TM_COL_SWEEP(false, kColStripNarrow);
        else
            TM_COL_SWEEP(false, kColStrip);
#undef TM_COL_SWEEP
    }
    return TM_OK;
}

// The fused step's arrays of one batch group (batches from b0 on).
struct FusedPtrs {
    const float *K;
    float *lv2, *lvw, *lse2_row, *log_u, *lu2, *log_v;
    const double *mu64, *nu64;
    double *lu64, *lv64;
    const uint8_t *inf_row, *inf_col;
    float2 *colpart;
};

FusedPtrs fused_ptrs(const SinkhornLayout &L, char *ws, float *log_u, float *log_v, int64_t b0) {
    const int64_t N = L.N, M = L.M;
    FusedPtrs P;
    P.K = reinterpret_cast<const float *>(ws + L.off_k) + b0 * N * M;
    P.lv2 = reinterpret_cast<float *>(ws + L.off_lv2) + b0 * M;
    P.lvw = reinterpret_cast<float *>(ws + L.off_lvw) + b0 * M;
    P.lse2_row = reinterpret_cast<float *>(ws + L.off_lse2row) + b0 * N;
    P.lu2 = reinterpret_cast<float *>(ws + L.off_lu2) + b0 * N;
    P.log_u = log_u + b0 * N;
    P.log_v = log_v + b0 * M;
    P.mu64 = reinterpret_cast<const double *>(ws + L.off_mu64) + b0 * N;
    P.nu64 = reinterpret_cast<const double *>(ws + L.off_nu64) + b0 * M;
    P.lu64 = reinterpret_cast<double *>(ws + L.off_lu64) + b0 * N;
    P.lv64 = reinterpret_cast<double *>(ws + L.off_lv64) + b0 * M;
    P.inf_row = reinterpret_cast<const uint8_t *>(ws + L.off_infrow) + b0 * N;
    P.inf_col = reinterpret_cast<const uint8_t *>(ws + L.off_infcol) + b0 * M;
    P.colpart = reinterpret_cast<float2 *>(ws + L.off_colpart) + b0 * (int64_t)L.fz_chunk * M;
    return P;
}

// The fused step runs when the row length has a shape and K (the start of
// the workspace) is 16-byte aligned; everything else it reads is in the
// workspace at 256-byte offsets.
bool fused_ok(const SinkhornLayout &L, const void *workspace) {
    return L.fused != kFzNone && ((uintptr_t)workspace % 16) == 0 && L.fz_chunk <= 0x7fffffff;
}

int launch_fused_step(const SinkhornLayout &L, bool exact, const FusedPtrs &P, double damp,
                      int ub, hipStream_t stream) {
    // TORCHMATCH_AMD_SINKHORN_SHIFT_WINDOW narrows the accepted |LSE - shift|
    // of rows and columns (base 2; default 16): "0" sends every row through
    // the exact two-pass and every column through the exact recompute, which
    // is how the tests reach those paths
    float win = kShiftWindow;
    if (const char *env = getenv("TORCHMATCH_AMD_SINKHORN_SHIFT_WINDOW"))
        win = fminf(kShiftWindow, fmaxf(0.f, (float)atof(env)));
    const float sum_lo = exp2f(-win), sum_hi = win > 0.f ? exp2f(win) : 0.f;
    const dim3 grid((unsigned)L.fz_chunk, (unsigned)L.B);
    const FusedShape &f = kFusedShapes[L.fused];
    // K past the 256 MiB Infinity Cache: streamed with non-temporal loads
    const bool nontemporal = (size_t)(L.B * L.N * L.M) * sizeof(float) > kNonTemporalBytes;
    const dim3 block(f.W * f.RW * 64);
#define TM_FUSED1(W_, RW_, NV_, NB_, EX_, NT_)                                             \
    TM_LAUNCH((sk_fused_step<W_, RW_, NV_, NB_, EX_, NT_>), grid, block, 0, stream, P.K,      \
              P.lv2, P.lvw, P.lse2_row, P.mu64, P.lu64, P.log_u, P.lu2,                             \
              P.colpart, L.N, L.M, L.fz_chunk, L.fz_rows, L.fz_interleave, sum_lo, sum_hi,   \
              damp, ub)
#define TM_FUSED(W_, RW_, NV_, NB_)                                                         \
    do {                                                                                    \
        if (exact && nontemporal)                                                           \
            TM_FUSED1(W_, RW_, NV_, NB_, true, true);                                       \
        else if (exact)                                                                     \
            TM_FUSED1(W_, RW_, NV_, NB_, true, false);                                      \
        else if (nontemporal)                                                               \
            TM_FUSED1(W_, RW_, NV_, NB_, false, true);                                      \
        else                                                                                \
            TM_FUSED1(W_, RW_, NV_, NB_, false, false);                                     \
    } while (0)
    switch (L.fused) {
    case kFz1x4x4: TM_FUSED(1, 4, 4, 1); break;
    case kFz1x4x8: TM_FUSED(1, 4, 8, 2); break;
    case kFz2x1x8: TM_FUSED(2, 1, 8, 1); break;
    case kFz4x1x8: TM_FUSED(4, 1, 8, 1); break;
    case kFz8x1x8: TM_FUSED(8, 1, 8, 2); break;
    case kFz16x1x4: TM_FUSED(16, 1, 4, 2); break;
    case kFz1x4x1: TM_FUSED(1, 4, 1, 2); break;
    case kFz1x4x2: TM_FUSED(1, 4, 2, 2); break;
    default: return TM_ERR_INTERNAL;
    }
#undef TM_FUSED
#undef TM_FUSED1
    const dim3 mgrid((unsigned)((L.M + 63) / 64), (unsigned)L.B);
    const MergeOut mo{P.lv64, P.log_v, P.lv2, P.lvw};
    // the column totals T_j are on the scale of the column marginals
    const double col_lo = win > 0.f ? 0x1p-96 : 1.0, col_hi = win > 0.f ? 0x1p96 : 0.0;
    if (L.fz_chunk > 64)  // C5: 256 chunks, 10.2 us with 16 waves against 11.3 with 4
        TM_LAUNCH(sk_col_merge_blk<16>, mgrid, dim3(16 * 64), 0, stream, P.colpart, P.K, P.lu2,
                  P.nu64, P.inf_col, mo, L.N, L.M, L.fz_chunk, exact ? 1 : 0, col_lo, col_hi,
                  damp, ub);
    else  // C4: 32 chunks, 5.0 us with 4 waves against 8.5 with 16
        TM_LAUNCH(sk_col_merge_blk<4>, mgrid, dim3(4 * 64), 0, stream, P.colpart, P.K, P.lu2,
                  P.nu64, P.inf_col, mo, L.N, L.M, L.fz_chunk, exact ? 1 : 0, col_lo, col_hi,
                  damp, ub);
    return TM_OK;
}

// ---- batch groups on side streams ------------------------------------------------
//
// The fused step of one batch depends only on that batch's previous step, so
// the batch can be split into groups that run their steps on separate streams:
// one group's merge launch and pass tail then overlap another group's pass.
// The side streams (default priority, non-blocking) and the fork / join events
// are created once per device (the device of the caller's stream) and kept
// until the process ends.  Every caller on a device shares them, so a caller
// holds the device's lock from the fork (event recorded on its stream, side
// streams wait on it) through its launches to the join (its stream waits on
// the side streams' events): another caller's fork can never land between
// them.  A stream under graph capture runs one group on that stream only, so
// the shared side streams are never pulled into a capture.
constexpr int kMaxGroups = 4;
constexpr int kMaxDevices = 64;

struct SideStreams {
    hipStream_t s[kMaxGroups - 1];
    hipEvent_t fork;
    hipEvent_t join[kMaxGroups - 1];
    bool ready;
    std::mutex mu;  // held across one fork -> launches -> join segment
};
SideStreams g_side[kMaxDevices];
std::mutex g_side_init_mu;

int side_streams(hipStream_t stream, SideStreams **out) {
    hipDevice_t dev = 0;
    if (hipStreamGetDevice(stream, &dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return TM_ERR_LAUNCH;
    std::lock_guard<std::mutex> lock(g_side_init_mu);
    SideStreams &ss = g_side[dev];
    if (!ss.ready) {
        int cur = 0;
        if (hipGetDevice(&cur) != hipSuccess)
            return TM_ERR_LAUNCH;
        if (cur != dev && hipSetDevice(dev) != hipSuccess)
            return TM_ERR_LAUNCH;
        bool ok = hipEventCreateWithFlags(&ss.fork, hipEventDisableTiming) == hipSuccess;
        for (int g = 0; ok && g < kMaxGroups - 1; ++g)
            ok = hipStreamCreateWithFlags(&ss.s[g], hipStreamNonBlocking) == hipSuccess &&
                 hipEventCreateWithFlags(&ss.join[g], hipEventDisableTiming) == hipSuccess;
        if (cur != dev && hipSetDevice(cur) != hipSuccess)
            ok = false;
        if (!ok)
            return TM_ERR_LAUNCH;
        ss.ready = true;
    }
    *out = &ss;
    return TM_OK;
}

bool stream_capturing(hipStream_t stream) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

// Batch groups for the fused step: two when B >= 2 (C4: 41.9 us per
// iteration against 50.2 on one stream; four groups 43-45 us).
// TORCHMATCH_AMD_SINKHORN_GROUPS overrides it (1 = the caller's stream only).
int fused_groups(const SinkhornLayout &L) {
    int64_t g = 2;
    if (const char *env = getenv("TORCHMATCH_AMD_SINKHORN_GROUPS"))
        g = atoi(env);
    if (g < 1)
        g = 1;
    if (g > kMaxGroups)
        g = kMaxGroups;
    return (int)(g < L.B ? g : L.B);
}

} // namespace

extern "C" int tm_sinkhorn_prepare_f32(const float *cost, const uint8_t *keep, const float *a,
                                       const float *b, int64_t B, int64_t N, int64_t M,
                                       float k_eps, void *workspace, size_t workspace_bytes,
                                       hipStream_t stream) {
    if (B < 0 || N < 0 || M < 0 || !(k_eps >= 0.f))
        return TM_ERR_INVALID_ARGUMENT;
    if (B == 0 || N == 0 || M == 0)
        return TM_OK;
    if (cost == nullptr || a == nullptr || b == nullptr)
        return TM_ERR_INVALID_ARGUMENT;
    const SinkhornLayout L = make_layout(B, N, M);
    if (workspace == nullptr || workspace_bytes < L.total)
        return TM_ERR_WORKSPACE;
    // prepare grid: y = row blocks of kPrepRows * groups rows (<= 65535)
    const int64_t row_groups = (N + kPrepRows - 1) / kPrepRows;
    const int64_t groups = (row_groups + 65534) / 65535;
    if (!shape_supported(L) || groups > 0x7fffffff)
        return TM_ERR_UNSUPPORTED_SHAPE;
    char *ws = static_cast<char *>(workspace);
    float *K = reinterpret_cast<float *>(ws + L.off_k);
    float *log_mu = reinterpret_cast<float *>(ws + L.off_logmu);
    float *log_nu = reinterpret_cast<float *>(ws + L.off_lognu);
    uint8_t *inf_row = reinterpret_cast<uint8_t *>(ws + L.off_infrow);
    uint8_t *inf_col = reinterpret_cast<uint8_t *>(ws + L.off_infcol);
    uint32_t *stats = reinterpret_cast<uint32_t *>(ws + L.off_stats);

    const int64_t n_flags = B * N > B * M ? B * N : B * M;
    TM_LAUNCH(sk_reset_flags, dim3(grid_for(n_flags, kMapBlock, 1 << 30)), dim3(kMapBlock), 0,
              stream, inf_row, B * N, inf_col, B * M, stats);
    double *mu64 = L.fused ? reinterpret_cast<double *>(ws + L.off_mu64) : nullptr;
    double *nu64 = L.fused ? reinterpret_cast<double *>(ws + L.off_nu64) : nullptr;
    TM_LAUNCH(sk_log_marginal, dim3(grid_for(B * N, kMapBlock, 1 << 30)), dim3(kMapBlock), 0,
              stream, a, log_mu, mu64, B * N, stats, kFlagANeg);
    TM_LAUNCH(sk_log_marginal, dim3(grid_for(B * M, kMapBlock, 1 << 30)), dim3(kMapBlock), 0,
              stream, b, log_nu, nu64, B * M, stats, kFlagBNeg);

    const bool vec = (M % 4) == 0 && ((uintptr_t)cost % 16) == 0 && ((uintptr_t)keep % 4) == 0;
    // the first step's K: base-2 when the iteration takes the fused step
    const double s2 = (fused_ok(L, workspace) && k_eps > 0.f) ? -kLog2eD / (double)k_eps : 0.0;
    const int cw = vec ? 4 : 1;
    const dim3 block(kPrepWaves * 64);
    const int g = (int)groups;
    for (int64_t b0 = 0; b0 < B; b0 += kBatchSlice) {
        const int64_t nb = B - b0 < kBatchSlice ? B - b0 : kBatchSlice;
        const int64_t eo = b0 * N * M;
        const float *c = cost + eo;
        const uint8_t *kp = keep != nullptr ? keep + eo : nullptr;
        uint8_t *ir = inf_row + b0 * N, *ic = inf_col + b0 * M;
        const dim3 grid((unsigned)((M + 64 * cw - 1) / (64 * cw)),
                        (unsigned)((row_groups + groups - 1) / groups), (unsigned)nb);
        if (vec && keep != nullptr)
            TM_LAUNCH((sk_prepare<true, true>), grid, block, 0, stream, c, kp, K + eo, ir, ic,
                      stats, N, M, g, k_eps, s2);
        else if (vec)
            TM_LAUNCH((sk_prepare<true, false>), grid, block, 0, stream, c, kp, K + eo, ir, ic,
                      stats, N, M, g, k_eps, s2);
        else if (keep != nullptr)
            TM_LAUNCH((sk_prepare<false, true>), grid, block, 0, stream, c, kp, K + eo, ir, ic,
                      stats, N, M, g, k_eps, s2);
        else
            TM_LAUNCH((sk_prepare<false, false>), grid, block, 0, stream, c, kp, K + eo, ir, ic,
                      stats, N, M, g, k_eps, s2);
    }
    return TM_OK;
}

extern "C" int tm_sinkhorn_read_stats(const void *workspace, int64_t B, int64_t N, int64_t M,
                                      uint32_t *flags, float *max_finite, hipStream_t stream) {
    if (flags == nullptr || max_finite == nullptr || B < 0 || N < 0 || M < 0)
        return TM_ERR_INVALID_ARGUMENT;
    *flags = 0;
    *max_finite = -INFINITY;
    if (B == 0 || N == 0 || M == 0)
        return TM_OK;
    if (workspace == nullptr)
        return TM_ERR_INVALID_ARGUMENT;
    const SinkhornLayout L = make_layout(B, N, M);
    uint32_t words[2] = {0, 0};
    if (hipMemcpyAsync(words, static_cast<const char *>(workspace) + L.off_stats, sizeof(words),
                       hipMemcpyDeviceToHost, stream) != hipSuccess)
        return TM_ERR_HIP;
    if (hipStreamSynchronize(stream) != hipSuccess)
        return TM_ERR_HIP;
    *flags = words[0];
    if (words[1] != 0) {
        const uint32_t k = words[1];
        const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
        float f;
        memcpy(&f, &u, sizeof(f));
        *max_finite = f;
        *flags |= TM_SK_FLAG_ANY_FINITE;
    }
    return TM_OK;
}

extern "C" int tm_sinkhorn_iterate_f32(const float *cost, const uint8_t *keep, int64_t B,
                                       int64_t N, int64_t M, const double *eps_sched,
                                       int32_t n_iter, double rho, float k_eps, float *log_plan,
                                       float *log_u, float *log_v, void *workspace,
                                       size_t workspace_bytes, hipStream_t stream) {
    if (B < 0 || N < 0 || M < 0 || n_iter < 1 || eps_sched == nullptr || !(k_eps >= 0.f))
        return TM_ERR_INVALID_ARGUMENT;
    for (int32_t s = 0; s < n_iter; ++s)
        if (!(eps_sched[s] > 0.0))
            return TM_ERR_INVALID_ARGUMENT;
    if (B == 0)
        return TM_OK;
    if (N == 0 || M == 0) {
        // no pair: every row and column is "all +inf", the potentials keep
        // their start value 0 (log_plan is empty)
        if (N > 0 && log_u != nullptr)
            TM_LAUNCH(sk_fill, dim3(grid_for(B * N, kMapBlock, 1 << 30)), dim3(kMapBlock), 0,
                      stream, log_u, B * N, 0.f);
        if (M > 0 && log_v != nullptr)
            TM_LAUNCH(sk_fill, dim3(grid_for(B * M, kMapBlock, 1 << 30)), dim3(kMapBlock), 0,
                      stream, log_v, B * M, 0.f);
        return TM_OK;
    }
    if (cost == nullptr || log_u == nullptr || log_v == nullptr)
        return TM_ERR_INVALID_ARGUMENT;
    const SinkhornLayout L = make_layout(B, N, M);
    if (workspace == nullptr || workspace_bytes < L.total)
        return TM_ERR_WORKSPACE;
    if (!shape_supported(L))
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
    const bool vec = (M % 4) == 0 && ((uintptr_t)log_v % 16) == 0;
    const bool fused = fused_ok(L, workspace);

    TM_LAUNCH(sk_fill, dim3(grid_for(B * N, kMapBlock, 1 << 30)), dim3(kMapBlock), 0, stream,
              log_u, B * N, 0.f);
    TM_LAUNCH(sk_fill, dim3(grid_for(B * M, kMapBlock, 1 << 30)), dim3(kMapBlock), 0, stream,
              log_v, B * M, 0.f);
    if (fused) {
        // float64 potentials and their scaled float32 copies start at 0; no
        // column shift yet (the first step folds exactly)
        const FusedPtrs P = fused_ptrs(L, ws, log_u, log_v, 0);
        const dim3 gn(grid_for(B * N, kMapBlock, 1 << 30)), gm(grid_for(B * M, kMapBlock, 1 << 30));
        TM_LAUNCH(sk_fill64, gn, dim3(kMapBlock), 0, stream, P.lu64, B * N, 0.0);
        TM_LAUNCH(sk_fill64, gm, dim3(kMapBlock), 0, stream, P.lv64, B * M, 0.0);
        TM_LAUNCH(sk_fill, gn, dim3(kMapBlock), 0, stream, P.lu2, B * N, 0.f);
        TM_LAUNCH(sk_fill, gm, dim3(kMapBlock), 0, stream, P.lv2, B * M, 0.f);
        TM_LAUNCH(sk_fill, gm, dim3(kMapBlock), 0, stream, P.lvw, B * M, 1.f);
    }

    const int64_t waves_per_batch = (N + kRowsPerWave - 1) / kRowsPerWave;
    const int64_t row_waves = B * waves_per_batch;
    const dim3 row_grid((unsigned)((row_waves + kRowWaves - 1) / kRowWaves));
    float cur_eps = k_eps > 0.f ? k_eps : -1.f;  // the epsilon K currently holds
    if (fused) {
        // steps run in segments of one epsilon (K rebuilt on the caller's
        // stream before a segment); within a segment each batch group runs its
        // steps on its own stream
        const int G = stream_capturing(stream) ? 1 : fused_groups(L);
        SideStreams *ss = nullptr;
        if (G > 1) {
            const int rc = side_streams(stream, &ss);
            if (rc != TM_OK)
                return rc;
        }
        for (int32_t s0 = 0; s0 < n_iter;) {
            const float e = (float)eps_sched[s0];
            bool exact0 = s0 == 0;
            if (e != cur_eps) {
                const int rc = launch_log_kernel(cost, keep, K, nK, e, true, stream);
                if (rc != TM_OK)
                    return rc;
                cur_eps = e;
                exact0 = true;
            }
            int32_t s1 = s0 + 1;
            while (s1 < n_iter && (float)eps_sched[s1] == e)
                ++s1;
            std::unique_lock<std::mutex> segment;
            if (G > 1) {
                segment = std::unique_lock<std::mutex>(ss->mu);
                if (hipEventRecord(ss->fork, stream) != hipSuccess)
                    return TM_ERR_LAUNCH;
                for (int g = 1; g < G; ++g)
                    if (hipStreamWaitEvent(ss->s[g - 1], ss->fork, 0) != hipSuccess)
                        return TM_ERR_LAUNCH;
            }
            int rc = TM_OK;
            for (int32_t s = s0; s < s1 && rc == TM_OK; ++s) {
                const double damp = unbalanced ? 1.0 / (1.0 + eps_sched[s] / rho) : 1.0;
                for (int g = 0; g < G && rc == TM_OK; ++g) {
                    // group g: batches [b0, b1), launched in slices
                    const int64_t b0 = g * L.B / G, b1 = (g + 1) * L.B / G;
                    for (int64_t c0 = b0; c0 < b1 && rc == TM_OK; c0 += kBatchSlice) {
                        SinkhornLayout Lg = L;
                        Lg.B = b1 - c0 < kBatchSlice ? b1 - c0 : kBatchSlice;
                        rc = launch_fused_step(Lg, s == s0 && exact0,
                                               fused_ptrs(L, ws, log_u, log_v, c0), damp,
                                               unbalanced ? 1 : 0,
                                               g == 0 ? stream : ss->s[g - 1]);
                    }
                }
            }
            // join the side streams even after a failed launch
            for (int g = 1; g < G; ++g)
                if (hipEventRecord(ss->join[g - 1], ss->s[g - 1]) != hipSuccess ||
                    hipStreamWaitEvent(stream, ss->join[g - 1], 0) != hipSuccess)
                    rc = TM_ERR_LAUNCH;
            if (rc != TM_OK)
                return rc;
            s0 = s1;
        }
    }
    for (int32_t s = 0; s < n_iter && !fused; ++s) {
        const float e = (float)eps_sched[s];
        if (e != cur_eps) {  // K holds -C / e for the step's epsilon
            const int rc = launch_log_kernel(cost, keep, K, nK, e, false, stream);
            if (rc != TM_OK)
                return rc;
            cur_eps = e;
        }
        const float damp = unbalanced ? (float)(1.0 / (1.0 + eps_sched[s] / rho)) : 1.f;
        if (vec) {
            const int64_t chunks = (M / 4 + 64 * kRowNV - 1) / (64 * kRowNV);
            const dim3 split_grid((unsigned)(B * N));
            const int ub = unbalanced ? 1 : 0;
            if (chunks <= 1)
                TM_LAUNCH(sk_row_sweep, row_grid, dim3(kRowWaves * 64), 0, stream, K, log_v,
                          log_mu, inf_row, log_u, B, N, M, waves_per_batch, damp, ub);
            else
                TM_LAUNCH((sk_row_sweep_split<8, 4>), split_grid, dim3(8 * 64), 0, stream, K,
                          log_v, log_mu, inf_row, log_u, N, M, damp, ub);
            const int rc = launch_col_sweep(L, true, K, log_u, log_nu, inf_col, log_v, colpart,
                                            damp, unbalanced ? 1 : 0, stream);
            if (rc != TM_OK)
                return rc;
        } else {
            TM_LAUNCH(sk_row_sweep_scalar, dim3(grid_for(B * N, 4, 1 << 30)), dim3(256), 0,
                      stream, K, log_v, log_mu, inf_row, log_u, B, N, M, damp,
                      unbalanced ? 1 : 0);
            const int rc = launch_col_sweep(L, false, K, log_u, log_nu, inf_col, log_v,
                                            colpart, damp, unbalanced ? 1 : 0, stream);
            if (rc != TM_OK)
                return rc;
        }
        if (L.n_chunk > 1)
            TM_LAUNCH(sk_col_merge, dim3(grid_for(B * M, kMapBlock, 1 << 30)), dim3(kMapBlock),
                      0, stream, colpart, log_nu, inf_col, log_v, B, M, L.n_chunk, damp,
                      unbalanced ? 1 : 0);
    }
    if (log_plan != nullptr && fused) {
        const FusedPtrs P = fused_ptrs(L, ws, log_u, log_v, 0);
        const float e_final = (float)eps_sched[n_iter - 1];
        const int pvec = (M % 4) == 0 && ((uintptr_t)cost % 16) == 0 &&
                         ((uintptr_t)keep % 4) == 0 && ((uintptr_t)log_plan % 16) == 0;
        const dim3 pgrid(grid_for(pvec ? nK / 4 : nK, kMapBlock, 8192));
        if (keep != nullptr)
            TM_LAUNCH(sk_plan64<true>, pgrid, dim3(kMapBlock), 0, stream, cost, keep, P.lu64,
                      P.lv64, log_plan, B, N, M, e_final, pvec);
        else
            TM_LAUNCH(sk_plan64<false>, pgrid, dim3(kMapBlock), 0, stream, cost, keep, P.lu64,
                      P.lv64, log_plan, B, N, M, e_final, pvec);
    } else if (log_plan != nullptr) {
        if (vec && ((uintptr_t)log_plan % 16) == 0)
            TM_LAUNCH(sk_plan4, dim3(grid_for(nK / 4, kMapBlock, 8192)), dim3(kMapBlock), 0,
                      stream, K, log_u, log_v, log_plan, B, N, M);
        else
            TM_LAUNCH(sk_plan, dim3(grid_for(nK, kMapBlock, 8192)), dim3(kMapBlock), 0, stream,
                      K, log_u, log_v, log_plan, B, N, M);
    }
    return TM_OK;
}

#undef TM_LAUNCH

extern "C" int tm_sinkhorn_f32(const float *cost, const float *a, const float *b, int64_t B,
                               int64_t N, int64_t M, const double *eps_sched, int32_t n_iter,
                               double rho, float *log_plan, float *log_u, float *log_v,
                               void *workspace, size_t workspace_bytes, hipStream_t stream) {
    if (B < 0 || N < 0 || M < 0 || n_iter < 1 || eps_sched == nullptr)
        return TM_ERR_INVALID_ARGUMENT;
    for (int32_t s = 0; s < n_iter; ++s)
        if (!(eps_sched[s] > 0.0))
            return TM_ERR_INVALID_ARGUMENT;
    const float k_eps = (float)eps_sched[0];
    const int rc = tm_sinkhorn_prepare_f32(cost, nullptr, a, b, B, N, M, k_eps, workspace,
                                           workspace_bytes, stream);
    if (rc != TM_OK)
        return rc;
    return tm_sinkhorn_iterate_f32(cost, nullptr, B, N, M, eps_sched, n_iter, rho, k_eps,
                                   log_plan, log_u, log_v, workspace, workspace_bytes, stream);
}
