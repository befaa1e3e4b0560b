// jv_batch.hip -- batched Jonker-Volgenant (float32) for gfx950.
//
// Reproduces the int64 row->col mapping of torchmatch's CPU
// `assignment::jonker_dense_batch` bit for bit, and that of
// `assignment::jonker_compact_batch` (section 3 below; K > 64 runs in
// jv_large.hip):
//   sentinel + padding      sources/torchmatch/assignment/cpu/ops.cpp:67-93,176-289
//   solver                  sources/torchmatch/assignment/cpu/jonker_dense_flat.h:27-274
//   compact solver          sources/torchmatch/assignment/cpu/jonker_compact_core.h:20-252
//
// Launch structure (one stream, no host round trip between kernels):
//   1. jv_stats_kernel     -- grid-stride pass over all B*N*M cells; each block
//                             writes {max finite, min finite, flags} to its own
//                             slot of a small workspace (no atomics, no memset).
//   2. jv_solve_kernel     -- one problem per 64-lane workgroup.  The block
//                             folds the per-block partials into the batch-global
//                             sentinel (max_finite+1)*(K+1), loads its K x K tile
//                             (padding 0, +inf -> sentinel) into LDS and into
//                             registers (lane j keeps column j), and runs the
//                             solver with one column / one cols[] position per
//                             lane.  Block 0 publishes the NaN / -inf flags.
//
// The wave-parallel solver follows the reference step by step; parallelism is
// only across columns, never across steps:
//   * column reduction: lane-serial column minima, LDS atomics for the
//     reverse-order claim, one wave-min per unique row for reduction transfer;
//   * augmenting row reduction: one wave-wide (min, second min) per step, the
//     first-index tie rule recovered with ballots;
//   * augmenting paths: lane p holds cols[p] and the state of that column.
//     find_dense / scan_dense swap cols[] entries in a fixed order; the swap
//     positions are found with a prefix-min scan and ballots, and the swaps are
//     replayed in that order, which gives exactly the sequential layout.
// Inputs whose magnitudes reach 1e15 (where the solver's LARGE = 1e18
// guards could become active) take a lane-serial transcription of the same
// algorithm instead, so the mapping stays exact for every finite input.
#include <hip/hip_runtime.h>
#include <math.h>
#include <atomic>
#include <mutex>
#include <vector>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "jv_batch.h"
#include "jv_common.h"
#include "jv_compact.h"
#include "wave.h"

namespace tmamd {
namespace {

constexpr int kTile = 64;                // K <= 64 path
constexpr int kStatsBlock = 1024;  // 16 waves: four per SIMD while the pass streams

// ---------------------------------------------------------------------------
// 1. statistics pass
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kStatsBlock)
jv_stats_kernel(const float *__restrict__ costs, int64_t n, JvStats *__restrict__ partial,
                uint32_t *__restrict__ status, uint32_t *__restrict__ replays) {
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        status[1] = 0;  // internal-error word, raised by jv_solve_kernel
        *replays = 0;   // problems the certified path handed to the exact replay
    }
    // Branch-free per value: the finite range as order-preserving integer
    // keys (no canonicalising float max / min; a -0.0 ranks just below
    // +0.0), the rare classes as lane masks on the scalar unit.
    constexpr int kKeyNegInf = (int)0x807fffff, kKeyPosInf = 0x7f800000;
    int kmx = kKeyNegInf, kmn = kKeyPosInf;
    uint64_t m_nan = 0, m_pinf = 0, m_ninf = 0, m_nz = 0;
    const int64_t stride = (int64_t)gridDim.x * kStatsBlock;
    const int64_t n4 = ((uintptr_t)costs % 16 == 0) ? n / 4 : 0;
    const float4 *c4 = reinterpret_cast<const float4 *>(costs);
    auto visit = [&](float x) {
        const uint32_t b = __float_as_uint(x);
        const int k = (int)(b ^ ((uint32_t)((int)b >> 31) & 0x7fffffffu));
        const bool fin = (b & 0x7f800000u) != 0x7f800000u;
        kmx = max(kmx, fin ? k : kKeyNegInf);
        kmn = min(kmn, fin ? k : kKeyPosInf);
        m_nan |= ballot((b & 0x7fffffffu) > 0x7f800000u);
        m_pinf |= ballot(b == 0x7f800000u);
        m_ninf |= ballot(b == 0xff800000u);
        m_nz |= ballot(b == 0x80000000u);
    };
    int64_t k0 = (int64_t)blockIdx.x * kStatsBlock + threadIdx.x;
    // four loads in flight per lane before any is folded (C2: each lane's
    // whole share of the 16 MiB in one round)
    constexpr int kInFlight = 4;
    for (; k0 + (kInFlight - 1) * stride < n4; k0 += kInFlight * stride) {
        float4 q[kInFlight];
#pragma unroll
        for (int u = 0; u < kInFlight; ++u)
            q[u] = c4[k0 + u * stride];
#pragma unroll
        for (int u = 0; u < kInFlight; ++u) {
            visit(q[u].x);
            visit(q[u].y);
            visit(q[u].z);
            visit(q[u].w);
        }
    }
    for (; k0 < n4; k0 += stride) {
        const float4 q = c4[k0];
        visit(q.x);
        visit(q.y);
        visit(q.z);
        visit(q.w);
    }
    for (int64_t k = n4 * 4 + (int64_t)blockIdx.x * kStatsBlock + threadIdx.x; k < n;
         k += stride)
        visit(costs[k]);

    // the keys back to floats (an involution on the bit patterns; no finite
    // value leaves -inf / +inf, as before)
    float mx = __int_as_float(kmx ^ ((kmx >> 31) & 0x7fffffff));
    float mn = __int_as_float(kmn ^ ((kmn >> 31) & 0x7fffffff));
    mx = wave_max(mx);
    mn = wave_min(mn);
    uint32_t f = (m_nan ? kJvFlagNan : 0u) | (m_pinf ? kJvFlagPosInf : 0u) |
                 (m_ninf ? kJvFlagNegInf : 0u) | (m_nz ? kJvFlagNegZero : 0u) |
                 (mx != -finf() ? kJvFlagAnyFinite : 0u);

    __shared__ float s_mx[kStatsBlock / 64], s_mn[kStatsBlock / 64];
    __shared__ uint32_t s_f[kStatsBlock / 64];
    const int w = threadIdx.x / 64;
    if (lane_id() == 0) {
        s_mx[w] = mx;
        s_mn[w] = mn;
        s_f[w] = f;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < kStatsBlock / 64; ++k) {
            mx = fmaxf(mx, s_mx[k]);
            mn = fminf(mn, s_mn[k]);
            f |= s_f[k];
        }
        partial[blockIdx.x].max_finite = mx;
        partial[blockIdx.x].min_finite = mn;
        partial[blockIdx.x].flags = f;
        partial[blockIdx.x].info = 0;
    }
}

// ---------------------------------------------------------------------------
// 2a. lane-serial transcription (exact for any finite input; slow)
// ---------------------------------------------------------------------------
struct SerialScratch {
    int32_t x[kTile], y[kTile], fr[kTile], pred[kTile], cols[kTile];
    float v[kTile], d[kTile];
    char unique[kTile];
};

__device__ uint32_t serial_find_tied(uint32_t n, uint32_t lo, const float *d, int32_t *cols) {
    uint32_t hi = lo + 1;
    float best = d[cols[lo]];
    for (uint32_t k = lo + 1; k < n; ++k) {
        const int32_t j = cols[k];
        const float dj = d[j];
        if (!(dj <= best))
            continue;
        if (dj < best) {
            best = dj;
            hi = lo;
        }
        cols[k] = cols[hi];
        cols[hi] = j;
        ++hi;
    }
    return hi;
}

__device__ int32_t serial_scan(uint32_t n, const float *c, uint32_t *plo, uint32_t *phi,
                               SerialScratch &s) {
    uint32_t lo = *plo, hi = *phi;
    while (lo != hi) {
        const int32_t jp = s.cols[lo++];
        const int32_t i = s.y[jp];
        const float level = s.d[jp];
        const float *row = c + i * kTile;
        const float h = row[jp] - s.v[jp] - level;
        for (uint32_t k = hi; k < n; ++k) {
            const int32_t j = s.cols[k];
            const float r = row[j] - s.v[j] - h;
            if (!(r < s.d[j]))
                continue;
            s.d[j] = r;
            s.pred[j] = i;
            if (r == level) {
                if (s.y[j] < 0)
                    return j;
                s.cols[k] = s.cols[hi];
                s.cols[hi] = j;
                ++hi;
            }
        }
    }
    *plo = lo;
    *phi = hi;
    return -1;
}

__device__ void serial_solve(uint32_t n, const float *c, SerialScratch &s) {
    for (uint32_t k = 0; k < n; ++k) {
        s.unique[k] = 1;
        s.x[k] = -1;
        s.v[k] = kLarge;
        s.y[k] = 0;
    }
    for (uint32_t i = 0; i < n; ++i)
        for (uint32_t j = 0; j < n; ++j)
            if (c[i * kTile + j] < s.v[j]) {
                s.v[j] = c[i * kTile + j];
                s.y[j] = (int32_t)i;
            }
    for (int32_t j = (int32_t)n - 1; j >= 0; --j) {
        const int32_t i = s.y[j];
        if (s.x[i] < 0) {
            s.x[i] = j;
        } else {
            s.unique[i] = 0;
            s.y[j] = -1;
        }
    }
    int32_t n_free = 0;
    for (uint32_t i = 0; i < n; ++i) {
        if (s.x[i] < 0) {
            s.fr[n_free++] = (int32_t)i;
        } else if (s.unique[i]) {
            const int32_t own = s.x[i];
            float mn = kLarge;
            for (uint32_t j = 0; j < n; ++j) {
                if ((int32_t)j == own)
                    continue;
                const float r = c[i * kTile + j] - s.v[j];
                if (r < mn)
                    mn = r;
            }
            s.v[own] -= mn;
        }
    }
    for (int round = 0; n_free > 0 && round < 2; ++round) {
        uint32_t cur = 0, rr = 0;
        int32_t still = 0;
        while (cur < (uint32_t)n_free) {
            ++rr;
            const int32_t fi = s.fr[cur++];
            const float *row = c + fi * kTile;
            int32_t j1 = 0, j2 = -1;
            float u1 = row[0] - s.v[0], u2 = kLarge;
            for (uint32_t j = 1; j < n; ++j) {
                const float r = row[j] - s.v[j];
                if (!(r < u2))
                    continue;
                if (r >= u1) {
                    u2 = r;
                    j2 = (int32_t)j;
                } else {
                    u2 = u1;
                    j2 = j1;
                    u1 = r;
                    j1 = (int32_t)j;
                }
            }
            int32_t i0 = s.y[j1];
            const float lowered = s.v[j1] - (u2 - u1);
            const bool lowers = lowered < s.v[j1];
            if (rr < cur * n) {
                if (lowers) {
                    s.v[j1] = lowered;
                } else if (i0 >= 0 && j2 >= 0) {
                    j1 = j2;
                    i0 = s.y[j2];
                }
                if (i0 >= 0) {
                    if (lowers)
                        s.fr[--cur] = i0;
                    else
                        s.fr[still++] = i0;
                }
            } else if (i0 >= 0) {
                s.fr[still++] = i0;
            }
            s.x[fi] = j1;
            s.y[j1] = fi;
        }
        n_free = still;
    }
    for (int32_t f = 0; f < n_free; ++f) {
        const int32_t start = s.fr[f];
        uint32_t lo = 0, hi = 0, n_ready = 0;
        int32_t final_j = -1;
        for (uint32_t j = 0; j < n; ++j) {
            s.cols[j] = (int32_t)j;
            s.d[j] = c[start * kTile + j] - s.v[j];
            s.pred[j] = start;
        }
        while (final_j < 0) {
            if (lo == hi) {
                n_ready = lo;
                hi = serial_find_tied(n, lo, s.d, s.cols);
                for (uint32_t k = lo; k < hi; ++k)
                    if (s.y[s.cols[k]] < 0)
                        final_j = s.cols[k];
            }
            if (final_j < 0)
                final_j = serial_scan(n, c, &lo, &hi, s);
        }
        const float level = s.d[s.cols[lo]];
        for (uint32_t k = 0; k < n_ready; ++k)
            s.v[s.cols[k]] += s.d[s.cols[k]] - level;
        int32_t j = final_j, i;
        uint32_t steps = 0;
        do {
            i = s.pred[j];
            s.y[j] = i;
            const int32_t prev = s.x[i];
            s.x[i] = j;
            j = prev;
            if (++steps >= n)
                break;
        } while (i != start);
    }
}

// ---------------------------------------------------------------------------
// 2b. wave-parallel solver, K <= 64
// ---------------------------------------------------------------------------

// Exchange the per-position state of lanes a and b (a != b, both uniform).
struct PosState {
    int col, pr, yc;
    float d, vc;
};

__device__ __forceinline__ void swap_lanes(PosState &st, int a, int b) {
    const int lane = lane_id();
    const int col_a = readlane_i(st.col, a), col_b = readlane_i(st.col, b);
    const int pr_a = readlane_i(st.pr, a), pr_b = readlane_i(st.pr, b);
    const int yc_a = readlane_i(st.yc, a), yc_b = readlane_i(st.yc, b);
    const float d_a = readlane_f(st.d, a), d_b = readlane_f(st.d, b);
    const float v_a = readlane_f(st.vc, a), v_b = readlane_f(st.vc, b);
    if (lane == a) {
        st.col = col_b;
        st.pr = pr_b;
        st.yc = yc_b;
        st.d = d_b;
        st.vc = v_b;
    } else if (lane == b) {
        st.col = col_a;
        st.pr = pr_a;
        st.yc = yc_a;
        st.d = d_a;
        st.vc = v_a;
    }
}

struct alignas(16) WaveLds {
    float c[kTile * kTile];  // row-major tile, stride 64
    int32_t xmax[kTile];     // column-reduction claims
    int32_t claims[kTile];
    float vbuf[kTile];       // column-indexed scatter buffers
    int32_t pbuf[kTile];
    double ubuf[kTile];      // certificate: row duals (float64)
    uint64_t adj[kTile];     // certificate: near-tight edges out of each column
};

// Two-minimum of one row (jonker_dense_flat.h:193-210): (u1, j1) is the
// first-index minimum; (u2, j2) the first-index minimum of the other columns,
// with the reference's starting slot (LARGE, -1) winning ties.  Requires the
// value at column 0 to be <= LARGE (the wave path guarantees it).  Ordering
// and ties use integer keys; u1 / u2 are the lanes' own float values.
struct TwoMin {
    int j1, j2;
    float u1, u2;
};

__device__ __forceinline__ TwoMin row_two_min(float r, bool live) {
    const int key = live ? fkey(r) : kKeyNone;
    int k1, k2;
    wave_min2_key(key, k1, k2);
    k1 = uniform_i(k1);
    k2 = uniform_i(k2);
    const uint64_t at1 = ballot(key == k1);
    TwoMin t;
    t.j1 = first_lane(at1);
    t.u1 = readlane_f(r, t.j1);
    int jj = -1;
    if (k2 == k1)
        jj = first_lane(at1 & (at1 - 1));
    else if (k2 != kKeyNone)
        jj = first_lane(ballot(key == k2));
    t.j2 = -1;
    t.u2 = kLarge;
    if (jj >= 0) {
        const float u = readlane_f(r, jj);
        if (u < kLarge) {
            t.u2 = u;
            t.j2 = jj;
        }
    }
    return t;
}

// Row cache of the augmenting row reduction (K >= 4).  Lane i keeps, for row
// i, the three columns that were its smallest reduced costs when the row was
// last scanned (ascending column order), their costs, the current duals and
// owners of those columns, and tau = the fourth smallest reduced cost of that
// scan.  Duals only fall in that phase, so every other reduced cost of the row
// is still >= tau.  When the second smallest cached value is < tau, the two
// cached minima are the row's two minima (first index on ties: the cached
// columns are compared in column order), and a step needs no row scan.  Every
// lane also keeps its row's would-be lowered dual, so a cached step reads all
// it needs from one lane.  A row never scanned has all values 0 and tau 0
// (reduced costs are >= 0 in that phase), so it is never taken as cached.
//
// The helpers take the cached entries by value: selecting among struct
// fields or captured references lets the compiler turn the selects into
// indexed private-memory loads.
struct CacheRank {
    int t1q, t1o;          // smallest: column, its owner
    float t1r, t2r, low;   // two smallest values, lowered dual of t1q
    uint64_t hitm, stepm;  // rows: cached / cached chain step
};

// Each row's two smallest cached values; the smallest's column is the first
// cached column holding it.  stepm: the row's step would lower the dual of an
// owned column (the reference's `free_rows[--current]` branch).
__device__ __forceinline__ CacheRank cache_rank(int q0, int q1, int q2, int o0, int o1, int o2,
                                                float g0, float g1, float g2, float w0,
                                                float w1, float w2, float tau) {
    CacheRank c;
    const float r0 = g0 - w0, r1 = g1 - w1, r2 = g2 - w2;
    c.t1r = fminf(fminf(r0, r1), r2);
    c.t2r = __builtin_amdgcn_fmed3f(r0, r1, r2);
    const bool e0 = r0 == c.t1r, e1 = r1 == c.t1r;
    c.t1q = e0 ? q0 : (e1 ? q1 : q2);
    const float t1w = e0 ? w0 : (e1 ? w1 : w2);
    c.t1o = e0 ? o0 : (e1 ? o1 : o2);
    c.low = t1w - (c.t2r - c.t1r);
    c.hitm = ballot(c.t2r < tau);
    c.stepm = c.hitm & ballot(c.low < t1w) & ballot(c.t1o >= 0);
    return c;
}

// Column of each row's second smallest cached value, (value, column) order.
__device__ __forceinline__ int cache_second(int q0, int q1, int q2, float g0, float g1,
                                            float g2, float w0, float w1, float w2,
                                            float t1r) {
    const float r0 = g0 - w0, r1 = g1 - w1, r2 = g2 - w2;
    const int not0 = r2 < r1 ? q2 : q1;
    const int not1 = r2 < r0 ? q2 : q0;
    const int not2 = r1 < r0 ? q1 : q0;
    return r0 == t1r ? not0 : (r1 == t1r ? not1 : not2);
}

// A fresh scan of one row (lane = column, `r` its reduced costs, `crow` its
// costs): the three smallest (value, column) in column order with their costs,
// duals and owners, and the fourth smallest value (K >= 4 live lanes).
struct CacheFill {
    int s0, s1, s2, oa, ob, oc;
    float ga, gb, gc, wa, wb, wc, tau;
};

__device__ __forceinline__ CacheFill cache_fill(float crow, float v, int y, bool live) {
    const int lane = lane_id();
    const int key = live ? fkey(crow - v) : kKeyNone;
    int k1, k2;
    wave_min2_key(key, k1, k2);
    // Usually exactly two lanes hold keys <= the second smallest, and they
    // are the first two in (value, column) order: drop them and take the
    // next two minima straight away.  Ties at the second value drop exactly
    // the first two lanes instead.
    int key3 = key <= k2 ? kKeyNone : key;
    int k3, k4;
    wave_min2_key(key3, k3, k4);
    uint64_t sel = ballot(key <= k2);
    if (__builtin_popcountll(sel) != 2) {
        const uint64_t m1 = ballot(key == k1);
        const uint64_t m2 = ballot(key == k2);
        const int j1 = first_lane(m1);
        const int j2 =
            uniform_i(k1) == uniform_i(k2) ? first_lane(m1 & (m1 - 1)) : first_lane(m2);
        key3 = (lane == j1 || lane == j2) ? kKeyNone : key;
        wave_min2_key(key3, k3, k4);
        sel = (1ull << j1) | (1ull << j2);
    }
    sel |= 1ull << first_lane(ballot(key3 == k3));
    CacheFill f;
    f.tau = key_to_float(k4);
    f.s0 = first_lane(sel);
    sel &= sel - 1;
    f.s1 = first_lane(sel);
    f.s2 = last_lane(sel);
    f.ga = readlane_f(crow, f.s0);
    f.gb = readlane_f(crow, f.s1);
    f.gc = readlane_f(crow, f.s2);
    f.wa = readlane_f(v, f.s0);
    f.wb = readlane_f(v, f.s1);
    f.wc = readlane_f(v, f.s2);
    f.oa = readlane_i(y, f.s0);
    f.ob = readlane_i(y, f.s1);
    f.oc = readlane_i(y, f.s2);
    return f;
}

// COMPACT = false: jonker_dense_flat.h:124-274 (jonker_dense_batch);
// COMPACT = true: jonker_compact_core.h:51-252 (jonker_compact_batch).  On the
// wave path's value range (every cost far below LARGE and FLT_MAX) the two
// solvers differ only in (a) the cap of the augmenting row reduction (none in
// the compact one), (b) which unassigned column of a minimum group ends a path
// (last / first), (c) the dual update's operand order, and (d) the starting
// minimum of the reduction transfer (LARGE / FLT_MAX, which only matters for
// K = 1); everything else is shared.
// Claim step of the column reduction (jonker_dense_flat.h:146-160): (v, y)
// arrive as this lane's column minimum and its first arg-min row; the
// highest column claiming a row keeps it.  On return y is the column's row
// (-1: free), x the lane's row's column (-1: free), lane k of fr the k-th free
// row (increasing), n_free their count; the result says whether the lane's
// row was claimed by one column only (the rows the transfer visits).
__device__ __forceinline__ bool column_claim(const int K, WaveLds &L, float &v, int &y, int &x,
                                             int &fr, int &n_free) {
    const int lane = lane_id();
    const bool live = lane < K;
    if (live) {
        L.xmax[lane] = -1;
        L.claims[lane] = 0;
    }
    __syncthreads();
    if (live) {
        atomicMax(&L.xmax[y], lane);
        atomicAdd(&L.claims[y], 1);
    }
    __syncthreads();
    x = live ? L.xmax[lane] : -1;                    // lane = row
    const bool unique_row = live ? (L.claims[lane] <= 1) : true;
    if (live && L.xmax[y] != lane)
        y = -1;                                      // lane = column
    if (!live) {
        v = finf();
        y = -1;
    }
    // lane k holds free_rows[k]: each free row writes itself at its rank
    const uint64_t m = ballot(live && x < 0);
    n_free = __builtin_popcountll(m);
    if ((m >> lane) & 1ull)
        L.pbuf[__builtin_popcountll(m & ((1ull << lane) - 1ull))] = lane;
    __syncthreads();
    fr = lane < n_free ? L.pbuf[lane] : 0;
    return unique_row;
}

// Column reduction of ccrrt_dense (jonker_dense_flat.h:124-176; the compact
// solver's jonker_compact_core.h:77-120 differs only in the transfer's
// starting minimum): the claim above, then the reduction transfer.  On
// return v holds the column duals after the transfer.
template <bool COMPACT, typename Row>
__device__ __forceinline__ void column_reduction(const int K, WaveLds &L, Row row, float &v,
                                                 int &y, int &x, int &fr, int &n_free) {
    const int lane = lane_id();
    const bool live = lane < K;
    const bool unique_row = column_claim(K, L, v, y, x, fr, n_free);
    // reduction transfer, unique rows in increasing order: each one sees
    // the v lowered by the rows before it; mn starts at LARGE and keeps
    // the first (lowest column) minimum, as the sequential scan does
    const float start_min = COMPACT ? kFltMax : kLarge;
    const int large_key = fkey(start_min);
    uint64_t t = ballot(live && x >= 0 && unique_row);
    while (t) {
        const int i = first_lane(t);
        t &= t - 1;
        const int own = readlane_i(x, i);
        const float r = row(i) - v;
        const int key = (live && lane != own) ? fkey(r) : kKeyNone;
        const int kmin = wave_min_key_s(key);
        float mn = start_min;
        if (kmin < large_key)
            mn = readlane_f(r, first_lane(ballot(key == kmin)));
        if (lane == own)
            v -= mn;
    }
}

// The same claim with the transfer done for every unique row at once, from
// the column minima (the duals before any transfer): lane i scans row i of
// the LDS tile, skewed by its own index so the lanes read different banks,
// and the row's column takes v -= min over the other columns of c - v.
// Every dual only falls, so each row's minimum taken from the earlier duals
// is at most its minimum under the final ones and the duals stay feasible
// (c - v >= the row's own reduced cost); the sequential transfer of the
// reference is one feasible choice among these.  For the certified path,
// whose answer does not depend on the starting duals.
__device__ __forceinline__ void column_reduction_parallel(const int K, WaveLds &L, float &v,
                                                          int &y, int &x, int &fr,
                                                          int &n_free, float start_min) {
    const int lane = lane_id();
    const bool live = lane < K;
    const bool unique_row = column_claim(K, L, v, y, x, fr, n_free);
    const bool transfer = live && x >= 0 && unique_row;
    // columns beyond K read as c - (-inf) = +inf and never win (their tile
    // entries are 0)
    L.vbuf[lane] = live ? v : -finf();
    __syncthreads();
    float mn = start_min;
    if (transfer) {
        const float4 *crow = reinterpret_cast<const float4 *>(L.c + lane * kTile);
        const float4 *vb = reinterpret_cast<const float4 *>(L.vbuf);
#pragma unroll
        for (int t = 0; t < kTile / 4; ++t) {
            const int q = (lane + t) & (kTile / 4 - 1);
            const float4 a = crow[q], b = vb[q];
            const int j = 4 * q;
            const float r0 = a.x - b.x, r1 = a.y - b.y, r2 = a.z - b.z, r3 = a.w - b.w;
            mn = (j != x && r0 < mn) ? r0 : mn;
            mn = (j + 1 != x && r1 < mn) ? r1 : mn;
            mn = (j + 2 != x && r2 < mn) ? r2 : mn;
            mn = (j + 3 != x && r3 < mn) ? r3 : mn;
        }
    }
    // column lane j takes the minimum of its row y_j
    const uint64_t moved = ballot(transfer);
    const int src = y < 0 ? lane : y;
    const float mrow = __int_as_float(__builtin_amdgcn_ds_bpermute(src * 4, __float_as_int(mn)));
    if (live && y >= 0 && ((moved >> y) & 1ull))
        v -= mrow;
}

template <bool COMPACT>
__device__ __forceinline__ bool wave_solve(const int K, WaveLds &L, float v,
                                           int y, bool chain, int &x_out) {
    const int lane = lane_id();
    const bool live = lane < K;

    // ---- column reduction (ccrrt_dense, jonker_dense_flat.h:124-176) ----
    int x, fr, n_free;
    column_reduction<COMPACT>(K, L, [&L, lane](int i) { return L.c[i * kTile + lane]; }, v, y,
                              x, fr, n_free);

    // ---- augmenting row reduction (carr_dense, jonker_dense_flat.h:178-235) ----
    // iteration guard: the reference's loop ends long before this; tripping it
    // means a bug here, reported through the status word instead of spinning
    // (the compact reduction has no cap: its guard is a step budget, which
    // also stands in for the cap of the chains below)
    const uint32_t rr_limit =
        COMPACT ? compact_arr_guard(K) : 4u * (uint32_t)K * (uint32_t)K * (uint32_t)K + 64u;
    // A general step follows the reference's branches with scalar selects.
    // When it displaces the previous owner of its column with a lowered dual
    // (the reference's `free_rows[--current] = i0`, almost every step on
    // uniform costs), the loop enters a displacement chain: the displaced
    // row's step is started before the previous step's outcome has reached
    // the scalar unit, and each step's updates are applied inside its own
    // argmin lane, gated there.  The first step that does not continue the
    // chain is handed back, untouched, to the general step.  x is not kept
    // during this phase; it is rebuilt from y afterwards (only assigned rows'
    // x are ever read again).
    //
    // row cache (see CacheRank above), lane = row
    const bool cache = chain && K >= 4;
    int q0 = kTile, q1 = kTile, q2 = kTile;  // cached columns
    int o0 = -1, o1 = -1, o2 = -1;           // their owners
    float g0 = 0.f, g1 = 0.f, g2 = 0.f;      // their costs in this row
    float w0 = 0.f, w1 = 0.f, w2 = 0.f;      // their duals
    float tau = 0.f;
    CacheRank rc = cache_rank(q0, q1, q2, o0, o1, o2, g0, g1, g2, w0, w1, w2, tau);
    for (int round = 0; n_free > 0 && round < 2; ++round) {
        uint32_t cur = 0, rr = 0;
        int still = 0;
        bool have = false;  // fi already known (handed back by a chain)
        int fi = 0;
        while (true) {
            if (!have) {
                if (cur >= (uint32_t)n_free)
                    break;
                fi = readlane_i(fr, (int)cur);
                have = true;
            }
            if (cache) {
                // ---- cached displacement chain ----
                // Steps that take the `free_rows[--current]` branch (cap, dual
                // lowered, column owned) run here from the cache alone: such a
                // step leaves `current` where it was, so fi stays pending at
                // position cur.  A row without a usable cache is rescanned
                // first.  The first step that is not such a step goes to the
                // general step below.
                const uint32_t rr_cap = COMPACT ? rr_limit : (cur + 1) * (uint32_t)K;
                while (true) {
                    while (((rc.stepm >> fi) & 1ull) && rr + 1 < rr_cap) {
                        const int c1 = readlane_i(rc.t1q, fi);
                        const float low = readlane_f(rc.low, fi);
                        const int ic = readlane_i(rc.t1o, fi);
                        ++rr;
                        const bool m0 = q0 == c1, m1 = q1 == c1, m2 = q2 == c1;
                        w0 = m0 ? low : w0;
                        w1 = m1 ? low : w1;
                        w2 = m2 ? low : w2;
                        o0 = m0 ? fi : o0;
                        o1 = m1 ? fi : o1;
                        o2 = m2 ? fi : o2;
                        if (lane == c1) {
                            v = low;
                            y = fi;
                        }
                        rc = cache_rank(q0, q1, q2, o0, o1, o2, g0, g1, g2, w0, w1, w2, tau);
                        fi = ic;
                    }
                    if (rr + 1 >= rr_cap || ((rc.hitm >> fi) & 1ull))
                        break;
                    const CacheFill f = cache_fill(L.c[fi * kTile + lane], v, y, live);
                    if (lane == fi) {
                        q0 = f.s0;
                        q1 = f.s1;
                        q2 = f.s2;
                        o0 = f.oa;
                        o1 = f.ob;
                        o2 = f.oc;
                        g0 = f.ga;
                        g1 = f.gb;
                        g2 = f.gc;
                        w0 = f.wa;
                        w1 = f.wb;
                        w2 = f.wc;
                        tau = f.tau;
                    }
                    rc = cache_rank(q0, q1, q2, o0, o1, o2, g0, g1, g2, w0, w1, w2, tau);
                    if (!((rc.stepm >> fi) & 1ull))
                        break;
                }
            }
            have = false;
            ++rr;
            ++cur;
            if (rr > rr_limit)
                return false;
            int j1, j2;
            float u1, u2;
            const bool hit = cache && ((rc.hitm >> fi) & 1ull);
            if (hit) {
                // u2 < tau < LARGE: the (LARGE, -1) start slot cannot win
                j1 = readlane_i(rc.t1q, fi);
                u1 = readlane_f(rc.t1r, fi);
                j2 = readlane_i(cache_second(q0, q1, q2, g0, g1, g2, w0, w1, w2, rc.t1r), fi);
                u2 = readlane_f(rc.t2r, fi);
            } else {
                const float r = L.c[fi * kTile + lane] - v;
                const int key = live ? fkey(r) : kKeyNone;
                int k1, k2;
                wave_min2_key(key, k1, k2);
                const uint64_t m1 = ballot(key == k1);
                const uint64_t m2 = ballot(key == k2);
                const bool same = uniform_i(k1) == uniform_i(k2);
                j1 = first_lane(m1);
                const uint64_t m1b = m1 & (m1 - 1);
                const int j2c =
                    same ? (m1b ? first_lane(m1b) : -1) : (m2 ? first_lane(m2) : -1);
                u1 = readlane_f(r, j1);
                const float u2c = readlane_f(r, j2c < 0 ? 0 : j2c);
                // (LARGE, -1) start slot of the second minimum
                const bool has2 = j2c >= 0 && u2c < kLarge;
                j2 = has2 ? j2c : -1;
                u2 = has2 ? u2c : kLarge;
            }
            const int j2r = j2 < 0 ? 0 : j2;
            const int i0 = readlane_i(y, j1);
            const int y2 = readlane_i(y, j2r);
            const float vj1 = readlane_f(v, j1);
            const float lowered = vj1 - (u2 - u1);
            const bool lowers = lowered < vj1;
            const bool cap = COMPACT || rr < cur * (uint32_t)K;
            const bool vupd = cap && lowers;
            const bool swap2 = cap && !lowers && i0 >= 0 && j2 >= 0;
            const int jsel = swap2 ? j2 : j1;
            const int isel = swap2 ? y2 : i0;
            const bool push_front = vupd && i0 >= 0;
            const bool push_back = !vupd && isel >= 0;
            if (vupd && lane == j1)
                v = lowered;
            if (push_back && lane == still)
                fr = isel;
            if (lane == jsel)
                y = fi;
            still += push_back ? 1 : 0;
            if (cache) {
                if (vupd) {
                    w0 = q0 == j1 ? lowered : w0;
                    w1 = q1 == j1 ? lowered : w1;
                    w2 = q2 == j1 ? lowered : w2;
                }
                o0 = q0 == jsel ? fi : o0;
                o1 = q1 == jsel ? fi : o1;
                o2 = q2 == jsel ? fi : o2;
                rc = cache_rank(q0, q1, q2, o0, o1, o2, g0, g1, g2, w0, w1, w2, tau);
            }
            if (!push_front)
                continue;
            // fr[--cur] = i0 is read straight back: keep i0 in a register
            --cur;
            fi = i0;
            have = true;
            if (!chain || cache)
                continue;

            // ---- displacement chain ----
            // Reduced costs are >= +0 throughout this phase (v starts at the
            // column minima and only falls), so their raw bits order them and
            // the second minimum's bits are its value.  A step continues the
            // chain when the reference would take its `free_rows[--current]`
            // branch: cap (rr_cnt < current * n, current counted after the
            // read), dual lowered, column owned.  Anything else ends the chain
            // and the general step above redoes that step exactly.
            const uint32_t rr_cap = COMPACT ? rr_limit : (cur + 1) * (uint32_t)K;
            uint64_t okm;
            int inext;
            float cnext;  // row of the displaced owner, loaded ahead
            {
                const float rc = L.c[fi * kTile + lane] - v;
                const int kc = live ? __float_as_int(rc) : kKeyNone;
                int c1, c2;
                wave_min2_key(kc, c1, c2);
                const int jc = first_lane(ballot(kc == c1));
                inext = readlane_i(y, jc);
                cnext = L.c[(inext & (kTile - 1)) * kTile + lane];
                const float lowc = v - (__int_as_float(c2) - rc);
                const bool okc = lane == jc && rr + 1 < rr_cap && lowc < v && y >= 0;
                if (okc) {
                    v = lowc;
                    y = fi;
                }
                okm = ballot(okc);
            }
            while (true) {
                // the displaced row, started before okm is consulted
                const int fn = inext & (kTile - 1);
                const float rn = cnext - v;
                const int kn = live ? __float_as_int(rn) : kKeyNone;
                int n1, n2;
                wave_min2_key(kn, n1, n2);
                const int jn = first_lane(ballot(kn == n1));
                const int inn = readlane_i(y, jn);
                cnext = L.c[(inn & (kTile - 1)) * kTile + lane];
                if (okm == 0)
                    break;  // fi's step leaves the chain: the general step redoes it
                ++rr;       // fi's step is committed (its ++current / --current cancel)
                fi = fn;
                const float lown = v - (__int_as_float(n2) - rn);
                const bool okn = lane == jn && rr + 1 < rr_cap && lown < v && y >= 0;
                if (okn) {
                    v = lown;
                    y = fi;
                }
                okm = ballot(okn);
                inext = inn;
            }
        }
        n_free = still;
    }
    // x from y: every assigned column names its row (free rows keep -1;
    // the augmentation below overwrites them before reading)
    if (live)
        L.xmax[lane] = -1;
    __syncthreads();
    if (live && y >= 0)
        L.xmax[y] = lane;
    __syncthreads();
    x = live ? L.xmax[lane] : -1;
    __syncthreads();

    // ---- augmentation (ca_dense / find_path_dense, jonker_dense_flat.h:75-122,237-258) ----
    int pred_col = 0;   // lane = column
    for (int f = 0; f < n_free; ++f) {
        const int start = readlane_i(fr, f);
        PosState st;
        st.col = lane;
        st.d = live ? (L.c[start * kTile + lane] - v) : finf();
        st.pr = start;
        st.yc = y;
        st.vc = v;
        int lo = 0, hi = 0, n_ready = 0;
        int final_j = -1;
        float group_level = 0.f;
        while (final_j < 0) {
            if (lo >= K)
                return false;  // no unassigned column reachable: cannot happen
            if (lo == hi) {
                // find_dense over positions [lo, K): a new running minimum
                // swaps with position lo, a tie with it swaps with hi
                n_ready = lo;
                const bool act = live && lane >= lo;
                const int dkey = act ? fkey(st.d) : kKeyNone;
                const int before = wave_shift_up_key(wave_prefix_min_key(dkey));
                const bool later = act && lane > lo;
                const uint64_t rec = ballot(later && dkey < before);
                const uint64_t tie = ballot(later && dkey == before);
                uint64_t ev = rec | tie;
                hi = lo + 1;
                while (ev) {
                    const int k = first_lane(ev);
                    ev &= ev - 1;
                    if ((rec >> k) & 1ull) {
                        swap_lanes(st, k, lo);
                        hi = lo + 1;
                    } else {
                        if (k != hi)
                            swap_lanes(st, k, hi);
                        ++hi;
                    }
                }
                group_level = readlane_f(st.d, lo);
                const uint64_t open =
                    ballot(live && lane >= lo && lane < hi && st.yc < 0);
                // dense: the last unassigned column of the group ends the
                // path (jonker_dense_flat.h:96-103); compact: the first
                // (jonker_compact_core.h:200-206)
                if (open)
                    final_j = readlane_i(st.col, COMPACT ? first_lane(open) : last_lane(open));
            }
            if (final_j >= 0)
                break;
            // scan_dense: rows of the tied columns, one at a time
            int slo = lo, shi = hi;
            bool early = false;
            while (slo != shi) {
                const int q = slo++;
                const int jq = readlane_i(st.col, q);
                const int iq = readlane_i(st.yc, q);
                // the group's common d: compact uses the level of its
                // gathering, dense the scanned column's own d (equal values)
                const float level = COMPACT ? group_level : readlane_f(st.d, q);
                const float vq = readlane_f(st.vc, q);
                const float cq = L.c[iq * kTile + jq];
                const float h = cq - vq - level;
                const bool act = live && lane >= shi;
                const float cp = act ? L.c[iq * kTile + st.col] : 0.f;
                const float r = cp - st.vc - h;
                const bool better = act && r < st.d;
                const bool tie = better && r == level;
                const uint64_t ret = ballot(tie && st.yc < 0);
                if (ret) {
                    const int kk = first_lane(ret);
                    // compact stops before relaxing column kk itself (only its
                    // pred is set); that d is never read again either way
                    if (better && (COMPACT ? lane < kk : lane <= kk))
                        st.d = r;
                    if (better && lane <= kk)
                        st.pr = iq;
                    final_j = readlane_i(st.col, kk);
                    early = true;
                    break;
                }
                if (better) {
                    st.d = r;
                    st.pr = iq;
                }
                uint64_t tm = ballot(tie);
                while (tm) {
                    const int k = first_lane(tm);
                    tm &= tm - 1;
                    if (k != shi)
                        swap_lanes(st, k, shi);
                    ++shi;
                }
            }
            if (!early) {
                lo = slo;
                hi = shi;
            }
        }
        // dual update of the columns made ready before the last level
        const float level = readlane_f(st.d, lo);
        if (live && lane < n_ready)
            st.vc = COMPACT ? (st.vc + st.d) - level : st.vc + (st.d - level);
        if (live) {
            L.vbuf[st.col] = st.vc;
            L.pbuf[st.col] = st.pr;
        }
        __syncthreads();
        if (live) {
            v = L.vbuf[lane];
            pred_col = L.pbuf[lane];
        }
        __syncthreads();
        // flip the assignment along the predecessor chain
        int j = final_j, i;
        int steps = 0;
        do {
            i = readlane_i(pred_col, j);
            if (lane == j)
                y = i;
            const int prev = readlane_i(x, i);
            if (lane == i)
                x = j;
            j = prev;
            if (++steps >= K)
                break;
        } while (i != start);
    }
    x_out = x;
    return true;
}

// ---------------------------------------------------------------------------
// 2c. certified shortest augmenting paths (square tiles of finite costs)
// ---------------------------------------------------------------------------
// The reference's augmenting row reduction (carr_dense) is a sequential chain
// whose length varies widely (C2 seed 0: 1,729 steps on the slowest problem,
// 240 at the median), and a batch waits for its slowest problem.  When the
// optimum is unique, every exact solver returns it, so this path runs the
// reference's column reduction, skips the row reduction and goes straight to
// one shortest augmenting path per free row (find_path_dense arithmetic,
// jonker_dense_flat.h:75-122, with one column picked per step instead of the
// reference's tie blocks), then proves its assignment x is the unique
// optimum by a margin:
//
//   u_i = c[i][x_i] - v[x_i] and r_ij = (c_ij - u_i) - v_j in float64 (exact
//   to ~1e-16 of the costs; r_{i x_i} = 0).  Any assignment s costs
//   cost(x) + sum_i r_{i s(i)}.  If every r_ij >= 0 and the graph with an
//   edge x_i -> j for each j != x_i with r_ij <= tau has no cycle, each cycle
//   of s x^-1 holds an edge with r > tau: every other assignment costs more
//   than cost(x) + tau.
//
// tau = 2^-20 S, S the largest |cost| of the problem (8 float32 ulps of S).
// Measured on the CPU against an exact float64 Hungarian solver, the float32
// reference returned the exact optimum on all 90,000 continuous-cost problems
// (mismatches only on exact ties), so no other answer is open to it when the
// margin holds.  A problem that fails the certificate (ties, near-ties, a
// negative reduced cost) is solved again by the exact replay of the
// reference's order (wave_solve / serial_solve).  C2 uniform costs: ~1 in
// 3,000 problems replays.  Returns false for "replay".
template <bool COMPACT>
__device__ __forceinline__ bool certified_solve(const int K, WaveLds &L, const Col64 &col,
                                                float v, int y, float tau, int &x_out) {
    const int lane = lane_id();
    const bool live = lane < K;
    int x, fr, n_free;
    column_reduction_parallel(K, L, v, y, x, fr, n_free, COMPACT ? kFltMax : kLarge);

    // One shortest path per free row.  Lane j holds column j: its distance d,
    // its order key (kKeyNone once scanned, and on dead lanes), its
    // predecessor row and its cost column in registers (col.get(i) = c[i][j],
    // an indexed VGPR move).  The key of a distance is its raw bits: d >= 0
    // up to rounding, and a misorder among rounding-size negatives only picks
    // another column of the same distance.  Lane j also holds uy_j = u of the
    // row y_j that owns column j, u_i = c[i][x_i] - v[x_i] = c[y_j][j] - v[j]
    // (fixed during a search), so the step's offset h = u_i - level of the
    // scanned column's row is read from the scanned lane itself, alongside
    // that row's index, not from a lane the row index selects.
    int pred = 0;
    float uy = 0.f;
    auto refresh_u = [&]() { uy = (live && y >= 0 ? L.c[y * kTile + lane] : 0.f) - v; };
    refresh_u();
    // free rows from the highest index down: on C2-like batches (16 seeds of
    // 1024 problems, CPU count) the slowest problem's search takes 356 steps
    // on average against 371 in increasing order
    for (int f = n_free - 1; f >= 0; --f) {
        const int start = readlane_i(fr, f);
        float d = col.get(start) - v;
        int key = live ? __float_as_int(d) : kKeyNone;
        pred = start;
        int jf = -1;
        float level = 0.f;
        // each step retires one lane for good (its key becomes kKeyNone), so
        // the loop ends within K steps.  The step loop is placed at a fixed
        // offset from a 64-byte instruction-cache line (the padding runs once
        // per search): its speed otherwise moves by several percent with the
        // size of the code before it.  Three words past the line was the
        // fastest of the offsets 0-7 measured on the C2 batches (seed 0: 60.4
        // us per launch, against 65.3 at two words and 63.5 at none;
        // re-measure when the loop changes).
        asm volatile(".p2align 6\n\ts_nop 0\n\ts_nop 0\n\ts_nop 0" ::: "memory");
        while (true) {
            const int kmin = wave_min_key_s(key);
            if (kmin == kKeyNone)
                break;
            const int js = first_lane(ballot(key == kmin));
            level = __int_as_float(kmin);  // an open column's key is its distance's bits
            const int is = readlane_i(y, js);
            const float us = readlane_f(uy, js);
            if (is < 0) {
                jf = js;  // unassigned column: the path ends
                break;
            }
            // relax through row `is`: r = c[i][j] - v[j] - (u_i - level), as
            // scan_dense's c[i][j] - v[j] - h, associated so that each step
            // of the sum takes one scalar
            const float r = ((col.get(is) - v) - us) + level;
            // an open lane's key is its distance's bits, and a scanned or
            // dead lane's key, kKeyNone, is a NaN pattern, against which
            // r < key is false: one compare, no separate test of the key
            const bool upd = r < __int_as_float(key);
            d = upd ? r : d;
            pred = upd ? is : pred;
            const int nk = upd ? __float_as_int(r) : key;
            // the scanned lane retires through a scalar mask (made as soon
            // as js is known), so this last select takes no vector compare
            key = __builtin_amdgcn_inverse_ballot_w64(~(1ull << js)) ? nk : kKeyNone;
        }
        if (jf < 0)
            return false;
        // dual update of the scanned columns (v[j] += d[j] - level)
        if (live && key == kKeyNone)
            v += d - level;
        // flip the assignment along the predecessor chain
        int j = jf;
        for (int hop = 0; hop < K; ++hop) {
            const int i = readlane_i(pred, j);
            const int prev = readlane_i(x, i);
            y = lane == j ? i : y;
            x = lane == i ? j : x;
            if (i == start)
                break;
            j = prev;
        }
        refresh_u();
    }
    if (ballot(live && (x < 0 || y < 0)))
        return false;

    // certificate: u of each column's row goes to the LDS, then row by row
    // every lane forms r_ij for its column (float64); lane i collects the
    // near-tight columns of row i, and lane c then takes those of its row y_c
    // Rows >= K get u = -inf and lanes >= K v = -inf, so every entry outside
    // the K x K tile reads r = +inf (never tight, never negative) and the
    // loop needs no row or lane masks.
    const double ninf = -__builtin_inf();
    L.ubuf[live ? y : lane] = live ? (double)L.c[y * kTile + lane] - (double)v : ninf;
    __syncthreads();
    const double vd = live ? (double)v : ninf;
    const double td = (double)tau;
    uint64_t neg = 0;
    uint32_t row_lo = 0, row_hi = 0;  // lane i: near-tight columns of row i
#pragma unroll
    for (int i = 0; i < kTile; ++i) {
        // rows from K on read r = +inf; past the first 16-row boundary at or
        // beyond K they are not visited (nor loaded into `col`)
        if (i % 16 == 0 && i >= K)
            break;
        const double r = ((double)col.get(i) - L.ubuf[i]) - vd;
        neg |= ballot(r < 0.0);
        const uint64_t tight = ballot(r <= td);
        row_lo = writelane_i((int)(uint32_t)tight, i, row_lo);
        row_hi = writelane_i((int)(uint32_t)(tight >> 32), i, row_hi);
    }
    if (neg)
        return false;
    // the row's own column is tight (r = 0): not an edge
    uint64_t row_adj = ((uint64_t)row_hi << 32) | row_lo;
    if (live)
        row_adj &= ~(1ull << x);
    // lane c: the edges out of column c are those of its row y_c
    const int src = (live ? y : lane) * 4;
    const uint64_t adj =
        live ? ((uint64_t)(uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)(row_adj >> 32)) << 32) |
                   (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)(uint32_t)row_adj)
             : 0ull;
    // peel columns without a near-tight edge into the remaining set; a cycle
    // survives
    uint64_t alive = ballot(live);
    for (int it = 0; it <= K && alive; ++it) {
        const uint64_t sink = ballot(((alive >> lane) & 1ull) && (adj & alive) == 0ull);
        if (!sink)
            break;
        alive &= ~sink;
    }
    if (alive)
        return false;
    x_out = x;
    return true;
}

// ---------------------------------------------------------------------------
// 3. the solve kernel (dense and compact), K <= 64
// ---------------------------------------------------------------------------
// jonker_compact_core.h:51-252 solves the same padded square problem as the
// dense solver with its own tie and ordering rules (listed in jv_compact.h),
// so its mappings differ on ties.  wave_solve<true> above follows them on the
// wave path; inputs outside its range take compact_serial (jv_compact.h).

// Statistics of one 64 x 64 tile held as 16 float4 per lane, reduced over
// the wave: the flags of jv_stats_kernel and the largest / smallest finite
// value.  All-finite tiles (the usual case) take integer max / min folds of
// the raw bits; a tile holding +-inf or NaN takes the per-value path.
__device__ __forceinline__ void tile_stats_wide(const float4 (&q)[16], float &mx, float &mn,
                                                uint32_t &flags) {
    uint32_t amax_bits = 0;  // largest |x| as raw bits (>= 0x7f800000: inf or NaN)
    int smin_bits = 0x7fffffff;  // smallest raw bits as a signed int (INT_MIN: -0.0)
    float hi = -finf(), lo = finf();
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const float e[4] = {q[k].x, q[k].y, q[k].z, q[k].w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t u = __float_as_uint(e[t]);
            amax_bits = max(amax_bits, u & 0x7fffffffu);
            smin_bits = min(smin_bits, (int)u);
            hi = __builtin_elementwise_maximum(hi, e[t]);
            lo = __builtin_elementwise_minimum(lo, e[t]);
        }
    }
    const bool clean = !ballot(amax_bits >= 0x7f800000u);
    if (clean) {
        mx = wave_max(hi);
        mn = wave_min(lo);
        flags = kJvFlagAnyFinite | (ballot(smin_bits == (int)0x80000000) ? kJvFlagNegZero : 0u);
        return;
    }
    float fmx = -finf(), fmn = finf();
    uint32_t f = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const float e[4] = {q[k].x, q[k].y, q[k].z, q[k].w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float x = e[t];
            if (isnan(x)) {
                f |= kJvFlagNan;
            } else if (isinf(x)) {
                f |= (x < 0.f) ? kJvFlagNegInf : kJvFlagPosInf;
            } else {
                f |= kJvFlagAnyFinite;
                if (__float_as_uint(x) == 0x80000000u)
                    f |= kJvFlagNegZero;
                fmx = fmaxf(fmx, x);
                fmn = fminf(fmn, x);
            }
        }
    }
    mx = wave_max(fmx);
    mn = wave_min(fmn);
    flags = 0;
#pragma unroll
    for (int bit = 0; bit < 5; ++bit)
        if (ballot((f >> bit) & 1u))
            flags |= 1u << bit;
}

// Lane j's column of the LDS tile into registers, with its minimum and first
// arg-min row (strict '<' from LARGE, jonker_dense_flat.h:136-144) and the
// largest |value|.  FULL (K = 64) has no row tests: a run-time bound on the
// unrolled rows costs a scalar mask and a branch per row.
template <bool FULL>
__device__ __forceinline__ void load_columns(const int K, const WaveLds &L, Col64 &col,
                                             float &vmin, int &ymin, float &amax) {
    const int lane = lane_id();
    vmin = kLarge;
    ymin = 0;
    amax = 0.f;
#pragma unroll
    for (int i = 0; i < kTile; ++i) {
        const bool row = FULL || i < K;
        if (!FULL && i % 16 == 0 && i >= K)
            break;  // rows from here on are never read from `col`
        // rows K .. (the next multiple of 16) - 1 hold 0 in the tile
        const float val = L.c[i * kTile + lane];
        col.set(i, val);
        amax = fmaxf(amax, fabsf(val));
        if (row && val < vmin) {
            vmin = val;
            ymin = i;
        }
    }
}

// Launch modes of jv_solve_kernel.
//   kJvStandalone: after jv_stats_kernel; every workgroup folds its partials
//     (the batch statistics), block 0 publishes the flags, every problem is
//     solved here.
//   kJvFusedSolve: no statistics pass.  Each workgroup takes its own tile's
//     statistics and writes them to its record, and its summary byte (flags
//     and kJvRec* bits).  A tile
//     without +inf, NaN or -inf needs nothing batch-wide (the sentinel only
//     replaces +inf, and the wave paths' range tests concern the tile's own
//     values), so it is solved here; a tile with +inf is deferred.  Block 0
//     clears the guard word.
//   kJvFusedFinish: the launch after kJvFusedSolve.  Block 0 folds every
//     record into the status words and the replay count and, for a batch
//     holding NaN or -inf, writes -1 to every output.  Deferred problems fold
//     the records (the batch statistics of the standalone mode) and are solved
//     with the batch-wide sentinel; the other workgroups return at once.
enum JvMode { kJvStandalone = 0, kJvFusedSolve = 1, kJvFusedFinish = 2 };

// Block 0 of kJvFusedFinish: status words, replay count, -1 fill on error,
// from the summary bytes (B of them, read as 32-bit words, eight per lane in
// flight).
__device__ __forceinline__ void finish_records(const uint8_t *__restrict__ summary, int64_t B,
                                               int N, int64_t *__restrict__ out,
                                               uint32_t *__restrict__ status,
                                               uint32_t *__restrict__ replays) {
    const int lane = lane_id();
    const uint32_t *words = reinterpret_cast<const uint32_t *>(summary);
    const int64_t n_words = (B + 3) / 4;
    uint32_t f = 0, nrep = 0;
    for (int64_t w0 = lane; w0 < n_words; w0 += 64 * 8) {
        uint32_t w[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t k = w0 + 64 * u;
            w[u] = k < n_words ? words[k] : 0u;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t k = w0 + 64 * u;
            const int64_t valid = B - 4 * k;  // bytes of this word that belong to problems
            const uint32_t mask = valid >= 4 ? 0xffffffffu
                                  : valid <= 0 ? 0u : (1u << (8 * valid)) - 1u;
            const uint32_t x = w[u] & mask;
            f |= x;
            nrep += (uint32_t)__builtin_popcount(x & 0x40404040u);
        }
    }
    f |= f >> 16;
    f |= f >> 8;
    uint32_t bits = 0;
#pragma unroll
    for (int bit = 0; bit < 8; ++bit)
        if (ballot((f >> bit) & 1u))
            bits |= 1u << bit;
    nrep = (uint32_t)wave_sum_all((float)nrep);  // exact: at most 2^24 problems
    const uint32_t flags = bits & 0x1fu;
    if (lane == 0) {
        *replays = nrep;
        if (bits & kJvRecGuard)
            raise_guard(status);
    }
    if (flags & (kJvFlagNan | kJvFlagNegInf)) {
        for (int64_t k = lane; k < B * (int64_t)N; k += 64)
            out[k] = -1;
    }
    // the flags last, with the done bit when no deferred problem is left to
    // solve in this launch: the release orders every write above before it
    if (lane == 0)
        __hip_atomic_store(&status[0], flags | ((bits & kJvRecDeferred) ? 0u : kJvFlagDone),
                           __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// kJvFusedSolve with host_tags (host-mapped pinned words): problem b's
// summary byte also goes to host_tags[b] as (tag << 8) | byte, the
// workgroup's last write, so a host waiting for the launch can fold the
// batch itself as the tags arrive (tm_jv_dense_batch_f32_sync).
__device__ __forceinline__ void publish_tag(uint32_t *host_tags, int64_t b, uint32_t tag,
                                            uint32_t byte) {
    if (host_tags != nullptr)
        __hip_atomic_store(&host_tags[b], (tag << 8) | byte, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
}

// One problem per 64-lane workgroup; COMPACT selects the solver of
// assignment::jonker_compact_batch instead of jonker_dense_batch (same
// statistics, sentinel, padding and output rules, ops.cpp:176-289).  `stats`
// holds the statistics partials (kJvStandalone, n_stats of them) or the
// per-problem records (fused modes, B of them).
template <bool COMPACT, int MODE>
__global__ void __launch_bounds__(64)
jv_solve_kernel(const float *__restrict__ costs, int64_t B, int N, int M,
                JvStats *__restrict__ stats, int n_stats, uint8_t *__restrict__ summary,
                int64_t *__restrict__ out, uint32_t *__restrict__ status, int certify,
                uint32_t *__restrict__ replays, uint32_t *__restrict__ host_tags, uint32_t tag) {
    __shared__ WaveLds L;
    __shared__ SerialScratch S;
    const int lane = lane_id();
    const int K = N > M ? N : M;
    const int64_t b = blockIdx.x;
    int64_t *ob = out + b * N;

    if constexpr (MODE == kJvFusedFinish) {
        if (b == 0)
            finish_records(summary, B, N, out, status, replays);
        if ((summary[b] & kJvRecDeferred) == 0)
            return;
    }
    if constexpr (MODE == kJvFusedSolve) {
        if (b == 0 && lane == 0)
            status[1] = 0;  // raised by kJvFusedFinish only
    }

    float mx, mn;
    uint32_t flags;
    const float *src = costs + b * (int64_t)N * M;
    // Square 64 x 64 tiles: issue the whole 16 KiB tile as 16 float4 loads per
    // lane before folding the statistics, so the HBM latency overlaps the fold.
    const bool wide = N == kTile && M == kTile && ((uintptr_t)src % 16) == 0;
    float4 q[16];
    if (wide) {
        const float4 *src4 = reinterpret_cast<const float4 *>(src);
#pragma unroll
        for (int k = 0; k < 16; ++k)
            q[k] = src4[k * 64 + lane];
    }
    uint32_t info = 0;  // kJvFusedSolve: this problem's record bits
    if constexpr (MODE == kJvFusedSolve) {
        if (wide) {
            tile_stats_wide(q, mx, mn, flags);
        } else {
            // Other shapes: the tile goes to the LDS as loaded (0 outside the
            // N x M problem) in the same pass that folds the statistics, 16
            // rows of loads in flight at a time (clamped addresses, so every
            // load is unconditional), up to the first 16-row boundary at or
            // past K (load_columns reads those rows).  A tile that holds +-inf
            // or NaN leaves below without being used, so no value needs the
            // sentinel here.
            float fmx = -finf(), fmn = finf();
            uint32_t f = 0;
            const bool lane_in = lane < M;
            const int64_t lane_off = lane_in ? lane : M - 1;
            for (int i0 = 0; i0 < K; i0 += 16) {
                float raw[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    const int i = i0 + u < N ? i0 + u : N - 1;
                    raw[u] = src[(int64_t)i * M + lane_off];
                }
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    const int i = i0 + u;
                    const bool real = lane_in && i < N;
                    const float x = raw[u];
                    const bool nan = real && isnan(x);
                    const bool inf = real && isinf(x);
                    const bool fin = real && !isnan(x) && !isinf(x);
                    f |= nan ? kJvFlagNan : 0u;
                    f |= inf ? ((x < 0.f) ? kJvFlagNegInf : kJvFlagPosInf) : 0u;
                    f |= fin ? kJvFlagAnyFinite : 0u;
                    f |= (fin && __float_as_uint(x) == 0x80000000u) ? kJvFlagNegZero : 0u;
                    fmx = fin ? fmaxf(fmx, x) : fmx;
                    fmn = fin ? fminf(fmn, x) : fmn;
                    L.c[i * kTile + lane] = real ? x : 0.f;
                }
            }
            mx = wave_max(fmx);
            mn = wave_min(fmn);
            flags = 0;
#pragma unroll
            for (int bit = 0; bit < 5; ++bit)
                if (ballot((f >> bit) & 1u))
                    flags |= 1u << bit;
        }
        const bool bad = (flags & (kJvFlagNan | kJvFlagNegInf)) != 0;
        if (bad || (flags & kJvFlagPosInf)) {
            if (bad) {
                for (int i = lane; i < N; i += 64)
                    ob[i] = -1;
            }
            if (lane == 0) {
                const uint32_t byte = flags | (bad ? 0u : kJvRecDeferred);
                stats[b] = JvStats{mx, mn, flags, 0u};
                summary[b] = (uint8_t)byte;
                publish_tag(host_tags, b, tag, byte);
            }
            return;
        }
    } else {
        fold_stats(stats, n_stats, mx, mn, flags);
        if constexpr (MODE == kJvStandalone) {
            if (b == 0 && lane == 0)
                status[0] = flags;
        }
        if (flags & (kJvFlagNan | kJvFlagNegInf)) {
            for (int i = lane; i < N; i += 64)
                ob[i] = -1;
            return;
        }
    }
    // the record of a problem solved in kJvFusedSolve, written last
    auto finish = [&]() {
        if constexpr (MODE == kJvFusedSolve) {
            if (lane == 0) {
                stats[b] = JvStats{mx, mn, flags, 0u};
                summary[b] = (uint8_t)(flags | info);
                publish_tag(host_tags, b, tag, flags | info);
            }
        }
    };
    auto note_guard = [&]() {
        if constexpr (MODE == kJvFusedSolve)
            info |= kJvRecGuard;
        else if (lane == 0)
            raise_guard(status);
    };
    const bool any_finite = (flags & kJvFlagAnyFinite) != 0;
    const float sentinel = any_finite ? (mx + 1.0f) * (float)(K + 1) : 1.0f;
    const bool has_inf = (flags & kJvFlagPosInf) != 0;
    bool fast = true;
    if (any_finite && (mx > kFastRange || mn < -kFastRange))
        fast = false;
    if (has_inf && !(fabsf(sentinel) <= kFastRange))
        fast = false;

    // tile into LDS (padding 0, +inf -> sentinel); then lane j scans column j
    // for its minimum and first arg-min row (strict '<' from LARGE,
    // jonker_dense_flat.h:136-144)
    bool inf_here = false;  // this problem holds +inf (the sentinel is in the tile)
    if (MODE == kJvFusedSolve && !wide) {
        // stored with the statistics above (a tile solved in this mode holds
        // no +inf)
    } else if (wide && MODE == kJvFusedSolve) {
        // a tile solved in this mode holds no +inf: stored as loaded
#pragma unroll
        for (int k = 0; k < 16; ++k)
            reinterpret_cast<float4 *>(L.c)[k * 64 + lane] = q[k];
    } else if (wide) {
        auto fix = [&](float x) {
            const bool f = isfinite(x);
            inf_here |= !f;
            return f ? x : sentinel;
        };
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            float4 t = q[k];
            t.x = fix(t.x);
            t.y = fix(t.y);
            t.z = fix(t.z);
            t.w = fix(t.w);
            reinterpret_cast<float4 *>(L.c)[k * 64 + lane] = t;
        }
    } else {
        // up to the first 16-row boundary at or past K (load_columns reads
        // those rows; rows from K on hold 0)
        const int k16 = (K + 15) & ~15;
#pragma unroll 16
        for (int i = 0; i < k16; ++i) {
            float val = 0.f;
            if (i < N && lane < M) {
                val = src[(int64_t)i * M + lane];
                if (!isfinite(val)) {
                    val = sentinel;
                    inf_here = true;
                }
            }
            L.c[i * kTile + lane] = val;
        }
    }
    __syncthreads();
    // (lane j also keeps its column in registers for the certified path)
    float vmin, amax;
    int ymin;
    Col64 col;
    if (K == kTile)
        load_columns<true>(K, L, col, vmin, ymin, amax);
    else
        load_columns<false>(K, L, col, vmin, ymin, amax);

    int x = -1;
    // certified shortest paths first (square, finite, S in [1e-30, 1e15]);
    // the exact replay below when the certificate does not hold
    amax = wave_max(lane < K ? amax : 0.f);
    if (certify && fast && N == M && !ballot(inf_here) && amax >= 1e-30f &&
        amax <= kFastRange) {
        if (certified_solve<COMPACT>(K, L, col, vmin, ymin, amax * 0x1p-20f, x)) {
            if (lane < N)
                ob[lane] = (int64_t)x;
            finish();
            return;
        }
        if constexpr (MODE == kJvFusedSolve) {
            info |= kJvRecReplayed;
        } else {
            if (lane == 0)
                atomicAdd(replays, 1u);
        }
        x = -1;
    }
    if constexpr (COMPACT) {
        if (fast && compact_wave_range(any_finite, mx, mn, has_inf, sentinel)) {
            const bool chain = K >= 2 && (flags & kJvFlagNegZero) == 0;
            if (!wave_solve<true>(K, L, vmin, ymin, chain, x)) {
                note_guard();
                x = -1;
            }
        } else {
            const float *tile = L.c;
            auto cost = [tile](int i, int j) { return tile[i * kTile + j]; };
            bool ok = true;
            if (lane == 0)
                ok = compact_serial((uint32_t)K, cost, S.x, S.y, S.fr, S.pred, S.cols, S.v, S.d);
            if (!__builtin_amdgcn_readfirstlane((int)ok))
                note_guard();
            __syncthreads();
            if (lane < K)
                x = S.x[lane];
        }
    } else if (fast) {
        // displacement chains need K >= 2 and no -0.0 (their second minimum is
        // read back from its key, which maps -0.0 to +0.0)
        const bool chain = K >= 2 && (flags & kJvFlagNegZero) == 0;
        if (!wave_solve<false>(K, L, vmin, ymin, chain, x)) {
            note_guard();
            x = -1;
        }
    } else {
        if (lane == 0)
            serial_solve((uint32_t)K, L.c, S);
        __syncthreads();
        if (lane < K)
            x = S.x[lane];
    }
    if (lane < N)
        ob[lane] = (x >= 0 && x < M) ? (int64_t)x : (int64_t)-1;
    finish();
}

} // namespace
} // namespace tmamd

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
using namespace tmamd;

// Workspace: the count of problems the certified path handed to the exact
// replay at offset 0, then from kStatsOffset the statistics records: the
// per-block partials of jv_stats_kernel (at most kJvMaxStatBlocks), or, on
// the fused K <= 64 path (B <= kFusedMaxB), one record per problem.
constexpr size_t kStatsOffset = 256;
// Fused path: the summary bytes follow the records.
size_t summary_offset(int64_t records) { return kStatsOffset + sizeof(JvStats) * (size_t)records; }
// Largest batch the fused path takes: every deferred (+inf) problem folds all
// B records, so its cost grows with B * (number of deferred problems).
constexpr int64_t kFusedMaxB = 2048;

namespace {
bool fused_path(int64_t B, int32_t N, int32_t M) {
    const int K = N > M ? N : M;
    return K <= kTile && B <= kFusedMaxB;
}
} // namespace

namespace {
int64_t record_count(int64_t B, int32_t N, int32_t M) {
    return (fused_path(B, N, M) && B > kJvMaxStatBlocks) ? B : kJvMaxStatBlocks;
}
} // namespace

extern "C" size_t tm_jv_workspace_bytes(int64_t B, int32_t N, int32_t M) {
    const int64_t records = record_count(B, N, M);
    const size_t summary = fused_path(B, N, M) ? (size_t)((B + 15) / 16 * 16) : 0;
    return summary_offset(records) + summary;
}

namespace {
// Offset of the large-K prefill in the workspace (after the statistics
// records), or 0 when the shape has none.
size_t prefill_offset(int64_t B, int32_t N, int32_t M) {
    const int K = N > M ? N : M;
    if (B <= 0 || N <= 0 || M <= 0 || K <= kTile || K > jv_large_max_k() ||
        jv_large_prep_bytes(B, N, M) == 0)
        return 0;
    return (tm_jv_workspace_bytes(B, N, M) + 255) / 256 * 256;
}
} // namespace

extern "C" size_t tm_jv_workspace_bytes_prefill(int64_t B, int32_t N, int32_t M) {
    const size_t off = prefill_offset(B, N, M);
    return off == 0 ? tm_jv_workspace_bytes(B, N, M) : off + jv_large_prep_bytes(B, N, M);
}

namespace {
// TORCHMATCH_AMD_JV_CERTIFY=0 switches the certified path off (every problem
// then takes the exact replay of the reference's order).
int certify_enabled() {
    const char *env = getenv("TORCHMATCH_AMD_JV_CERTIFY");
    return (env != nullptr && strcmp(env, "0") == 0) ? 0 : 1;
}

uint32_t *replay_counter(void *workspace) { return static_cast<uint32_t *>(workspace); }

JvStats *stats_records(void *workspace) {
    return reinterpret_cast<JvStats *>(static_cast<char *>(workspace) + kStatsOffset);
}

// The launches of tm_jv_dense_batch_f32 / tm_jv_compact_batch_f32.  K <= 64
// with B <= kFusedMaxB: the fused solve launch, then the finishing launch (no
// pass over the input besides the solve's own read).  Otherwise the
// statistics pass, then the solve (K <= 64) or the large-K kernel.
template <bool COMPACT>
int jv_launch(const float *costs, int64_t B, int32_t N, int32_t M, int64_t *out,
              void *workspace, size_t workspace_bytes, uint32_t *d_status, hipStream_t stream,
              uint32_t *host_tags = nullptr, uint32_t tag = 0) {
    if (B < 0 || N < 0 || M < 0)
        return kTmErrInvalidArgument;
    if (B == 0 || N == 0 || M == 0)
        return kTmOk;  // caller fills -1
    const int K = N > M ? N : M;
    if (K > (COMPACT ? jv_compact_max_k() : jv_large_max_k()))
        return kTmErrUnsupportedShape;
    if (workspace_bytes < tm_jv_workspace_bytes(B, N, M) || workspace == nullptr ||
        d_status == nullptr)
        return kTmErrWorkspace;
    if (B > (int64_t)0x7fffffff)
        return kTmErrUnsupportedShape;
    JvStats *stats = stats_records(workspace);
    uint32_t *replays = replay_counter(workspace);
    const int certify = certify_enabled();
    if (fused_path(B, N, M)) {
        uint8_t *summary = static_cast<uint8_t *>(workspace) + summary_offset(record_count(B, N, M));
        hipLaunchKernelGGL((jv_solve_kernel<COMPACT, kJvFusedSolve>), dim3((unsigned)B), dim3(64),
                           0, stream, costs, B, N, M, stats, (int)B, summary, out, d_status,
                           certify, replays, host_tags, tag);
        if (host_tags != nullptr)  // the caller folds the tags, then finishes if needed
            return hipGetLastError() == hipSuccess ? kTmOk : kTmErrLaunch;
        hipLaunchKernelGGL((jv_solve_kernel<COMPACT, kJvFusedFinish>), dim3((unsigned)B),
                           dim3(64), 0, stream, costs, B, N, M, stats, (int)B, summary, out,
                           d_status, certify, replays, nullptr, 0u);
        return hipGetLastError() == hipSuccess ? kTmOk : kTmErrLaunch;
    }
    const int64_t n = B * (int64_t)N * M;
    int64_t blocks = (n / 4 + kStatsBlock - 1) / kStatsBlock;
    blocks = blocks < 1 ? 1 : (blocks > kJvMaxStatBlocks ? kJvMaxStatBlocks : blocks);
    hipLaunchKernelGGL(jv_stats_kernel, dim3((unsigned)blocks), dim3(kStatsBlock), 0, stream,
                       costs, n, stats, d_status, replays);
    if (hipGetLastError() != hipSuccess)
        return kTmErrLaunch;
    if (K > kTile) {
        // the prefill when the workspace holds it (the same result without)
        const size_t off = prefill_offset(B, N, M);
        void *prep = (off != 0 && workspace_bytes >= tm_jv_workspace_bytes_prefill(B, N, M))
                         ? static_cast<char *>(workspace) + off
                         : nullptr;
        return COMPACT ? launch_jv_compact_large(costs, B, N, M, stats, (int)blocks, prep, out,
                                                 d_status, stream)
                       : launch_jv_large(costs, B, N, M, stats, (int)blocks, prep, out,
                                         d_status, stream);
    }
    hipLaunchKernelGGL((jv_solve_kernel<COMPACT, kJvStandalone>), dim3((unsigned)B), dim3(64), 0,
                       stream, costs, B, N, M, stats, (int)blocks, nullptr, out, d_status,
                       certify, replays, nullptr, 0u);
    return hipGetLastError() == hipSuccess ? kTmOk : kTmErrLaunch;
}
} // namespace

extern "C" int tm_jv_read_replays(const void *workspace, uint32_t *count, hipStream_t stream) {
    if (workspace == nullptr || count == nullptr)
        return TM_ERR_INVALID_ARGUMENT;
    if (hipMemcpyAsync(count, workspace, sizeof(uint32_t), hipMemcpyDeviceToHost, stream) !=
        hipSuccess)
        return TM_ERR_HIP;
    return hipStreamSynchronize(stream) == hipSuccess ? TM_OK : TM_ERR_HIP;
}

extern "C" int tm_jv_dense_batch_f32(const float *costs, int64_t B, int32_t N, int32_t M,
                                     int64_t *out, void *workspace, size_t workspace_bytes,
                                     uint32_t *d_status, hipStream_t stream) {
    return jv_launch<false>(costs, B, N, M, out, workspace, workspace_bytes, d_status, stream);
}

extern "C" int tm_jv_compact_batch_f32(const float *costs, int64_t B, int32_t N, int32_t M,
                                       int64_t *out, void *workspace, size_t workspace_bytes,
                                       uint32_t *d_status, hipStream_t stream) {
    return jv_launch<true>(costs, B, N, M, out, workspace, workspace_bytes, d_status, stream);
}

// ---------------------------------------------------------------------------
// Synchronous entry points: the launch, the wait and the status in one call,
// for callers that wait for the result anyway (the torch ops).  On the fused
// path (K <= 64, B <= kFusedMaxB) every solve workgroup publishes its summary
// byte to host-mapped pinned memory under a tag unique to the call; the host
// folds them as they arrive, so a batch with no +inf, NaN or -inf needs no
// finishing launch and returns as soon as its last problem is solved.  Other
// batches run the finishing launch (deferred problems, the -1 fill) or the
// statistics-pass path, and the host synchronises the stream.
// ---------------------------------------------------------------------------
namespace {
// Pinned words: the two status words, then one tag word per problem
// (kFusedMaxB of them).  Blocks are allocated once per device and reused: a
// host thread takes one from its device's pool at its first call and hands it
// back when it exits, so the pinned memory held is one block per device per
// host thread alive at once (sizeof(uint32_t) * (2 + kFusedMaxB) = 8,200 bytes
// each), and a thread-per-request caller reuses blocks instead of allocating.
// The pool itself is never destroyed (a thread may exit during process
// teardown) and nothing is freed; the blocks go with the process.
struct HostWords {
    uint32_t *host = nullptr;
    uint32_t *dev = nullptr;
};

constexpr int kMaxDevices = 64;

struct HostWordsPool {
    std::mutex mu;
    std::vector<HostWords> free_blocks[kMaxDevices];
};

HostWordsPool &host_words_pool() {
    static HostWordsPool *pool = new HostWordsPool;  // leaked on purpose, see above
    return *pool;
}

// The calling thread's blocks, returned to the pool when the thread exits.
struct ThreadWords {
    HostWords slot[kMaxDevices];
    ~ThreadWords() {
        HostWordsPool &pool = host_words_pool();
        std::lock_guard<std::mutex> lock(pool.mu);
        for (int d = 0; d < kMaxDevices; ++d)
            if (slot[d].host != nullptr)
                pool.free_blocks[d].push_back(slot[d]);
    }
};

HostWords *host_words(hipStream_t stream) {
    thread_local ThreadWords mine;
    hipDevice_t dev = 0;
    if (hipStreamGetDevice(stream, &dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return nullptr;
    HostWords &w = mine.slot[dev];
    if (w.host != nullptr)
        return &w;
    HostWordsPool &pool = host_words_pool();
    {
        std::lock_guard<std::mutex> lock(pool.mu);
        if (!pool.free_blocks[dev].empty()) {
            w = pool.free_blocks[dev].back();
            pool.free_blocks[dev].pop_back();
            return &w;
        }
    }
    const size_t bytes = sizeof(uint32_t) * (2 + (size_t)kFusedMaxB);
    void *h = nullptr;
    void *d = nullptr;
    if (hipHostMalloc(&h, bytes, hipHostMallocMapped) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    if (hipHostGetDevicePointer(&d, h, 0) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipHostFree(h);
        return nullptr;
    }
    memset(h, 0, bytes);
    w.host = static_cast<uint32_t *>(h);
    w.dev = static_cast<uint32_t *>(d);
    return &w;
}

// 24-bit call tags, never 0 (the words' value when allocated).
uint32_t next_tag() {
    static std::atomic<uint32_t> counter{0};
    uint32_t t;
    do
        t = (counter.fetch_add(1, std::memory_order_relaxed) + 1u) & 0xffffffu;
    while (t == 0);
    return t;
}

template <bool COMPACT>
int jv_sync(const float *costs, int64_t B, int32_t N, int32_t M, int64_t *out,
            void *workspace, size_t workspace_bytes, uint32_t *replays_out,
            hipStream_t stream) {
    if (replays_out != nullptr)
        *replays_out = 0;
    if (B < 0 || N < 0 || M < 0)
        return kTmErrInvalidArgument;
    if (B == 0 || N == 0 || M == 0)
        return kTmOk;  // caller fills -1
    HostWords *hw = host_words(stream);
    if (hw == nullptr)
        return TM_ERR_HIP;
    volatile uint32_t *words = hw->host;
    words[0] = 0;
    words[1] = 0;
    if (!fused_path(B, N, M)) {
        const int rc = jv_launch<COMPACT>(costs, B, N, M, out, workspace, workspace_bytes,
                                          hw->dev, stream);
        // synchronise before returning, also after an error: the words are reused
        const hipError_t e = hipStreamSynchronize(stream);
        if (rc != kTmOk)
            return rc;
        if (e != hipSuccess)
            return TM_ERR_HIP;
        const uint32_t seen[2] = {words[0], words[1]};
        return tm_jv_status_code(seen);
    }
    // the tag words of this batch start at 0: a word left by an earlier call
    // (whose writes all landed before it returned) can then never carry the
    // new tag, even after the 24-bit tags wrap
    volatile uint32_t *tags = words + 2;
    for (int64_t p = 0; p < B; ++p)
        tags[p] = 0;
    const uint32_t tag = next_tag();
    int rc = jv_launch<COMPACT>(costs, B, N, M, out, workspace, workspace_bytes, hw->dev, stream,
                                hw->dev + 2, tag);
    if (rc != kTmOk) {
        (void)hipStreamSynchronize(stream);
        return rc;
    }
    // fold the tagged summaries as they arrive; if the stream goes idle
    // before all of them are in, the launch failed
    uint32_t acc = 0, nrep = 0;
    int64_t seen = 0;
    for (uint32_t spin = 1; seen < B; ++spin) {
        const uint32_t t = tags[seen];
        if ((t >> 8) == tag) {
            acc |= t & 0xffu;
            nrep += (t & kJvRecReplayed) ? 1u : 0u;
            ++seen;
            continue;
        }
        if ((spin & 4095u) == 0 && hipStreamQuery(stream) != hipErrorNotReady) {
            const hipError_t e = hipStreamSynchronize(stream);
            if ((tags[seen] >> 8) != tag)
                return e != hipSuccess ? TM_ERR_HIP : TM_ERR_INTERNAL;
        }
    }
    if (replays_out != nullptr)
        *replays_out = nrep;
    const uint32_t flags = acc & 0x1fu;
    if ((acc & kJvRecDeferred) || (flags & (kJvFlagNan | kJvFlagNegInf))) {
        // deferred problems and the -1 fill: the finishing launch
        uint8_t *summary =
            static_cast<uint8_t *>(workspace) + summary_offset(record_count(B, N, M));
        hipLaunchKernelGGL((jv_solve_kernel<COMPACT, kJvFusedFinish>), dim3((unsigned)B),
                           dim3(64), 0, stream, costs, B, N, M, stats_records(workspace), (int)B,
                           summary, out, hw->dev, certify_enabled(), replay_counter(workspace),
                           nullptr, 0u);
        rc = hipGetLastError() == hipSuccess ? kTmOk : kTmErrLaunch;
        const hipError_t e = hipStreamSynchronize(stream);
        if (rc != kTmOk)
            return rc;
        if (e != hipSuccess)
            return TM_ERR_HIP;
        const uint32_t st[2] = {words[0], words[1]};
        return tm_jv_status_code(st);
    }
    return (acc & kJvRecGuard) ? TM_ERR_INTERNAL : TM_OK;
}
} // namespace

extern "C" int tm_jv_dense_batch_f32_sync(const float *costs, int64_t B, int32_t N, int32_t M,
                                          int64_t *out, void *workspace, size_t workspace_bytes,
                                          uint32_t *replays, hipStream_t stream) {
    return jv_sync<false>(costs, B, N, M, out, workspace, workspace_bytes, replays, stream);
}

extern "C" int tm_jv_compact_batch_f32_sync(const float *costs, int64_t B, int32_t N,
                                            int32_t M, int64_t *out, void *workspace,
                                            size_t workspace_bytes, uint32_t *replays,
                                            hipStream_t stream) {
    return jv_sync<true>(costs, B, N, M, out, workspace, workspace_bytes, replays, stream);
}

// ---------------------------------------------------------------------------
// Entry point that allocates nothing (no counterpart in the reference): for
// callers that cannot allocate device memory (code under graph capture, tight
// serving loops).  Its workspace is `scratch`, a file-scope device array of a
// fixed size (each GPU the library runs on keeps its own copy until the
// process ends); every call on one GPU shares it, so calls that overlap on
// one GPU race.  Nothing in it needs clearing between calls: every record a
// launch reads is written earlier in the same call (each problem's record by
// its fused solve workgroup, or every partial by the statistics pass), and
// the guard word and the replay counter are set before they are raised or read.
// ---------------------------------------------------------------------------
namespace {
// >= tm_jv_workspace_bytes(B, N, M) for every shape: kFusedMaxB records and
// summary bytes
constexpr size_t kScratchBytes =
    kStatsOffset + (sizeof(JvStats) + 1) * (size_t)kFusedMaxB;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kScratchMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kScratchMaxDevices] = {};

// The device address of `scratch` on the device of `stream`, looked up once
// per device with that device current (in host code the array's name is not
// a device address).
int scratch_address(hipStream_t stream, void **out) {
    hipDevice_t dev = 0;
    if (hipStreamGetDevice(stream, &dev) != hipSuccess || dev < 0 || dev >= kScratchMaxDevices)
        return TM_ERR_HIP;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        int cur = 0;
        if (hipGetDevice(&cur) != hipSuccess)
            return TM_ERR_HIP;
        if (cur != dev && hipSetDevice(dev) != hipSuccess)
            return TM_ERR_HIP;
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev && hipSetDevice(cur) != hipSuccess)
            return TM_ERR_HIP;
        if (e != hipSuccess || p == nullptr)
            return TM_ERR_HIP;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return TM_OK;
}
} // namespace

extern "C" size_t tm_jv_noalloc_scratch_bytes(void) { return kScratchBytes; }

extern "C" int tm_jv_dense_batch_f32_noalloc(const float *costs, int64_t B, int32_t N,
                                             int32_t M, int64_t *out, uint32_t *d_status,
                                             hipStream_t stream) {
    if (B < 0 || N < 0 || M < 0)
        return kTmErrInvalidArgument;
    if (B == 0 || N == 0 || M == 0)
        return kTmOk;  // caller fills -1
    if (tm_jv_workspace_bytes(B, N, M) > kScratchBytes)
        return kTmErrWorkspace;
    void *ws = nullptr;
    const int rc = scratch_address(stream, &ws);
    if (rc != TM_OK)
        return rc;
    return tm_jv_dense_batch_f32(costs, B, N, M, out, ws, kScratchBytes, d_status, stream);
}

extern "C" int32_t tm_jv_max_k(void) { return jv_large_max_k(); }

extern "C" int32_t tm_jv_compact_max_k(void) { return jv_compact_max_k(); }

extern "C" int tm_jv_status_code(const uint32_t *h_status) {
    if (h_status == nullptr)
        return TM_ERR_INVALID_ARGUMENT;
    if (h_status[1] != 0)
        return TM_ERR_INTERNAL;
    if (h_status[0] & kJvFlagNan)
        return TM_ERR_NAN;
    if (h_status[0] & kJvFlagNegInf)
        return TM_ERR_NEG_INF;
    return TM_OK;
}

extern "C" int tm_jv_check_status(const uint32_t *d_status, hipStream_t stream) {
    uint32_t words[2] = {0, 0};
    if (hipMemcpyAsync(words, d_status, sizeof(words), hipMemcpyDeviceToHost, stream) !=
        hipSuccess)
        return TM_ERR_HIP;
    if (hipStreamSynchronize(stream) != hipSuccess)
        return TM_ERR_HIP;
    return tm_jv_status_code(words);
}
