// jv_large.hip -- batched Jonker-Volgenant for 64 < K <= 1024 (gfx950).
//
// Same contract as the K <= 64 kernel in jv_batch.hip: the int64 row->col
// mapping of torchmatch's CPU `jonker_dense_batch` bit for bit
// (sources/torchmatch/assignment/cpu/ops.cpp:176-289,
//  sources/torchmatch/assignment/cpu/jonker_dense_flat.h:27-274), and with
// COMPACT that of `jonker_compact_batch` (ops.cpp:431-433 around
// jonker_compact_core.h:20-252; its rules are listed in jv_compact.h).
//
// One 64-lane workgroup per problem.  A K x K tile no longer fits in LDS, so
// the cost is read from global memory (L2 / Infinity Cache) through a view
// that pads virtually (rows >= N and columns >= M read 0) and maps +inf to
// the batch sentinel -- the padded tile is never materialised.  Per-column
// state (v, y, d, pred), per-row state (x, the row cache), the free-row list
// and the cols[] permutation live in LDS (about 108 KiB).  Lane l handles
// columns / positions l, l + 64, l + 128, ... of every K-wide pass; passes
// that must respect the reference's sequential order (first index on ties,
// the swaps of find_dense and scan_dense) are resolved with per-chunk
// ballots in increasing index order, and the swap sequence itself is
// replayed by lane 0 on cols[] -- swaps are rare events, the K-wide
// relaxations around them are parallel.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "jv_batch.h"
#include "jv_common.h"
#include "jv_compact.h"
#include "wave.h"

namespace tmamd {
namespace {

constexpr int kMaxLargeK = 1024;   // with the row cache and the prefill
constexpr int kMaxChunks = kMaxLargeK / 64;
constexpr int kMaxXLK = 2048;      // beyond: no row cache (the state alone fills 80 KiB)
constexpr int kXLChunks = kMaxXLK / 64;
constexpr int kCacheSlots = 16;  // row-cache depth; one slot per lane of lanes 0..15
constexpr int kKeyLarge = __builtin_bit_cast(int, kLarge);  // fkey(kLarge): kLarge > 0

// The solve's LDS for K <= KMAX; SLOTS = 0: no row cache (its arrays are one
// row long and never touched).
template <int KMAX, int SLOTS>
struct LargeLdsT {
    static constexpr int kMax = KMAX;
    static constexpr int kSlots = SLOTS;
    float v[KMAX];
    float d[KMAX];
    float rbuf[KMAX];
    int32_t y[KMAX];
    int32_t x[KMAX];
    int32_t fr[KMAX];
    int32_t pred[KMAX];
    int32_t cols[KMAX];
    int32_t ev[KMAX];  // claims in the column reduction, swap events later
    int32_t emap[KMAX];  // position -> index in the current tie run, else -1
    // Row cache of the augmenting row reduction: for row i, up to
    // kCacheSlots columns that were its smallest reduced costs when it was
    // filled (ascending column order, -1 = empty slot), their costs, and tau
    // = the next smallest reduced cost of that fill (-inf: never filled).
    // Duals only fall from the column reduction on, so every other reduced
    // cost of the row is still >= tau; when the second smallest cached value
    // (with the current duals) is < tau, the two cached minima are the row's
    // two minima, first column on ties.  Filled with 16 columns for every
    // row before the solve when the caller's workspace holds the prefill
    // (jv_large_rowcache_kernel), and with 3 by the row scans.  Columns are
    // 16-bit (K <= 1024), so the 16-slot cache of 1024 rows takes 96 KiB.
    // On the C3 batch's slowest problem 16 prefilled slots leave 9 of its
    // 2,496 row-reduction steps to scan their row, 8 left 80 (CPU model of
    // the cache policy, which reproduces the kernel's counts).
    alignas(16) int16_t cq[SLOTS ? KMAX : 1][kCacheSlots];  // 16-byte copies (copy_to_lds)
    alignas(16) float cg[SLOTS ? KMAX : 1][kCacheSlots];
    float ctau[SLOTS ? KMAX : 1];
};
typedef LargeLdsT<kMaxLargeK, kCacheSlots> LargeLds;
typedef LargeLdsT<kMaxXLK, 0> LargeLdsXL;  // 64 < K <= 2048 without the cache: 80 KiB

// The virtually padded K x K tile: 0 outside (N, M), +inf -> sentinel.
struct CostView {
    const float *src;
    int N, M;
    float sentinel;
};

// Raw costs of a real row (i < N), lane l holding columns l, l + 64, ...
// Every lane loads every chunk (addresses clamped into the row, extra values
// ignored by the callers), so the loads carry no branches and all of them are
// in flight before any is used: a row costs one memory latency.
template <int NC>
__device__ __forceinline__ void load_row_raw(const CostView &C, int i, float (&raw)[NC]) {
    const int lane = lane_id();
    const float *src = C.src + (int64_t)i * C.M;
#pragma unroll
    for (int e = 0; e < NC; ++e)
        raw[e] = src[min(e * 64 + lane, C.M - 1)];
}

// The padded-tile view of a raw cost: +inf -> sentinel, columns >= M -> 0.
__device__ __forceinline__ float fix_cost(const CostView &C, float raw, int j) {
    return j >= C.M ? 0.f : (isfinite(raw) ? raw : C.sentinel);
}

// Row i of the padded tile into registers (values for j >= K are unused).
template <int NC>
__device__ __forceinline__ void load_row(const CostView &C, int i, float (&cr)[NC]) {
    const int lane = lane_id();
    if (i < C.N) {
        float raw[NC];
        load_row_raw<NC>(C, i, raw);
#pragma unroll
        for (int e = 0; e < NC; ++e)
            cr[e] = fix_cost(C, raw[e], e * 64 + lane);
    } else {
#pragma unroll
        for (int e = 0; e < NC; ++e)
            cr[e] = 0.f;
    }
}

// The solve's workgroup is one wave (64 threads): its LDS operations execute
// in issue order, so a sync between lanes only has to keep the compiler from
// moving LDS accesses across it.  Wavefront-scope fences around the wave
// barrier do that and emit no wait for outstanding LDS operations (a
// workgroup fence, as in __syncthreads, waits for all of them).
__device__ __forceinline__ void lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// A run of tie events: for i = 0 .. n-1 in order, swap cols[pos_i] with
// cols[h0 + i] (pos_i = ev[k0 + i], strictly increasing, pos_i >= h0 + i).
// The result, computed for all events at once: cols[h0 + i] receives the
// original cols[pos_i]; a position pos_i >= h0 + n receives what was at h0 + i
// when event i ran -- the original element there, unless h0 + i was an
// earlier event's position pos_j (j < i), in which case it is what event j
// received, and so on down the chain.  Leaves emap all -1.
template <class LDS>
__device__ void apply_tie_run(LDS &L, int k0, int n, int h0) {
    const int lane = lane_id();
    for (int i = lane; i < n; i += 64)
        L.emap[L.ev[k0 + i] & 0x7fffffff] = i;
    lds_sync();
    constexpr int kPer = LDS::kMax / 64;
    int a[kPer], b[kPer];
#pragma unroll
    for (int t = 0; t < kPer; ++t) {
        const int i = t * 64 + lane;
        if (i < n) {
            const int pos = L.ev[k0 + i] & 0x7fffffff;
            a[t] = L.cols[pos];
            if (pos >= h0 + n) {
                int h = h0 + i;
                int j = L.emap[h];
                while (j >= 0 && j < i) {  // j strictly falls: at most i steps
                    h = h0 + j;
                    j = L.emap[h];
                }
                b[t] = L.cols[h];
            }
        }
    }
    lds_sync();
#pragma unroll
    for (int t = 0; t < kPer; ++t) {
        const int i = t * 64 + lane;
        if (i < n) {
            const int pos = L.ev[k0 + i] & 0x7fffffff;
            L.cols[h0 + i] = a[t];
            if (pos >= h0 + n)
                L.cols[pos] = b[t];
        }
    }
    lds_sync();
    for (int i = lane; i < n; i += 64)
        L.emap[L.ev[k0 + i] & 0x7fffffff] = -1;
    lds_sync();
}

// Replays find_dense's swap events in order: bit 31 set = a new running
// minimum (swap with lo, hi back to lo + 1), clear = a tie (swap with hi, then
// hi + 1).  Each new minimum is one swap; each run of ties in between goes
// through apply_tie_run.  Returns hi (uniform).
template <class LDS>
__device__ int replay_find_events(LDS &L, int n_ev, int lo) {
    const int lane = lane_id();
    int hi = lo + 1;
    int k = 0;
    while (k < n_ev) {
        const int e = L.ev[k];
        if (e < 0) {
            const int pos = e & 0x7fffffff;
            lds_sync();
            if (lane == 0) {
                const int t = L.cols[pos];
                L.cols[pos] = L.cols[lo];
                L.cols[lo] = t;
            }
            lds_sync();
            hi = lo + 1;
            ++k;
            continue;
        }
        // the run of ties up to the next new minimum
        int r = n_ev;
        for (int base = k; base < n_ev; base += 64) {
            const int q = base + lane;
            const uint64_t recm = ballot(q < n_ev && L.ev[q] < 0);
            if (recm) {
                r = base + first_lane(recm);
                break;
            }
        }
        apply_tie_run(L, k, r - k, hi);
        hi += r - k;
        k = r;
    }
    return hi;
}

// Append the set bits of `mask` (positions base + lane) to L.ev in increasing
// order, tagged with `tag`; returns the new count (uniform).
template <class LDS>
__device__ __forceinline__ int append_events(LDS &L, int n_ev, uint64_t mask, int base,
                                             uint32_t tag_mask_rec, uint64_t rec_mask) {
    const int lane = lane_id();
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    if ((mask >> lane) & 1ull) {
        const int slot = n_ev + __builtin_popcountll(mask & below);
        const bool rec = (rec_mask >> lane) & 1ull;
        L.ev[slot] = (base + lane) | (rec ? (int)tag_mask_rec : 0);
    }
    return n_ev + __builtin_popcountll(mask);
}

// A row's costs, chunk e of lane l at [e]; a vector value, so a read at a
// wave-uniform chunk compiles to an indexed register move.
typedef float f32x16 __attribute__((ext_vector_type(kMaxChunks)));
typedef float f32x32 __attribute__((ext_vector_type(kXLChunks)));
template <int NC> struct ChunkVec { typedef f32x16 type; };
template <> struct ChunkVec<kXLChunks> { typedef f32x32 type; };

// Lane l's value of chunk e (e, l uniform).
template <class V>
__device__ __forceinline__ float chunk_value(const V &v, int e, int l) {
    return readlane_f(v[e], l);
}

// Smallest and second smallest key (as a multiset) of lanes 0..15, in each
// of those lanes: four pair-merge butterfly stages inside the 16-lane row.
__device__ __forceinline__ void min2_16_key(int key, int &k1, int &k2) {
    int a = key, b = kKeyNone;
    pair_merge(a, b, dpp_full<kDppQuadXor1>(a), dpp_full<kDppQuadXor1>(b));
    pair_merge(a, b, dpp_full<kDppQuadXor2>(a), dpp_full<kDppQuadXor2>(b));
    pair_merge(a, b, dpp_full<kDppRowHalfMirror>(a), dpp_full<kDppRowHalfMirror>(b));
    pair_merge(a, b, dpp_full<kDppRowMirror>(a), dpp_full<kDppRowMirror>(b));
    k1 = a;
    k2 = b;
}

// One problem's share of the prefill (all null: none).  v / y: the column
// reduction's minima and their rows (K each); cq / cg: kCacheSlots cache
// columns and costs per real row (N x kCacheSlots), ctau: their tau (N).
struct LargePrep {
    const float *v;
    const int32_t *y;
    const int16_t *cq;
    const float *cg;
    const float *ctau;
};

// n dwords from global memory into LDS, eight 16-byte loads per lane in
// flight (n % 4 == 0, both sides 16-byte aligned).  Loads and stores carry
// no condition (lanes past the end copy the last 16 bytes again), so the
// compiler cannot sink each load into a guarded store and wait for it alone.
__device__ __forceinline__ void copy_to_lds(void *dst, const void *src, int n) {
    const int lane = lane_id();
    const int n4 = n / 4;
    if (n4 <= 0)
        return;
    int4 *d = static_cast<int4 *>(dst);
    const int4 *q = static_cast<const int4 *>(src);
    for (int base = 0; base < n4; base += 8 * 64) {
        int4 t[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            t[u] = q[min(base + u * 64 + lane, n4 - 1)];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            d[min(base + u * 64 + lane, n4 - 1)] = t[u];
    }
}

// Smallest column j = e * 64 + lane with key kk[e] == k, other than x1 and
// x2 (uniform; kKeyNone if there is none).  One wave minimum over the
// columns: the first column in index order, as the reference's scans take it.
template <int NC>
__device__ __forceinline__ int first_column(const int (&kk)[NC], int k, int x1, int x2) {
    const int lane = lane_id();
    int best = kKeyNone;
#pragma unroll
    for (int e = NC - 1; e >= 0; --e) {
        const int j = e * 64 + lane;
        if (kk[e] == k && j != x1 && j != x2)
            best = j;
    }
    return wave_min_key_s(best);
}

// One row's two-minimum by a full scan (reference order: first column on
// ties, the (LARGE, -1) start slot of the second minimum, column 0 as the
// first seed).  When `refill` is set and the result is within LARGE, the row
// cache of fi is refilled from the same scan.  Nothing goes through LDS: the
// columns of the two (three) smallest come from wave minima over the column
// indices, their costs from the owning lanes.
template <int NC, class LDS>
__device__ void scan_row(LDS &L, const CostView &C, int fi, int E, int K,
                         bool refill, int &j1, int &j2, float &u1, float &u2) {
    const int lane = lane_id();
    typename ChunkVec<NC>::type cr;
    {
        float c[NC];
        load_row<NC>(C, fi, c);
#pragma unroll
        for (int e = 0; e < NC; ++e)
            cr[e] = c[e];
    }
    // reduced costs, lane-local two-minimum of keys (the duals are read
    // outside the guard, all in flight together: a read inside it would be
    // waited for chunk by chunk)
    int kk[NC];
    float vv[NC];
#pragma unroll
    for (int e = 0; e < NC; ++e)
        vv[e] = L.v[min(e * 64 + lane, K - 1)];
    int a = kKeyNone, bk = kKeyNone;
#pragma unroll
    for (int e = 0; e < NC; ++e) {
        const int j = e * 64 + lane;
        kk[e] = kKeyNone;
        if (e < E && j < K) {
            const float r = cr[e] - vv[e];
            const int k = fkey(r);
            kk[e] = k;
            if (k < a) {
                bk = a;
                a = k;
            } else if (k < bk) {
                bk = k;
            }
        }
    }
    int k1, k2;
    {
        int p1, p2;
        wave_min2_key(a, p1, p2);
        // the multiset two-minimum of the per-lane pairs: merge with b
        const int bmin = uniform_i(wave_min_key(bk));
        k1 = uniform_i(p1);
        k2 = min(uniform_i(p2), bmin);
    }
    // a reduced cost c - v, recomputed from the cost held by its lane
    auto reduced = [&](int j) { return chunk_value(cr, j >> 6, j & 63) - L.v[j]; };
    const float r0 = uniform_f(reduced(0));
    j1 = -1;
    j2 = -1;
    if (!(r0 <= kLarge)) {
        // the reference seeds (v1, j1) with column 0; beyond LARGE that seed
        // changes the outcome: run its scan verbatim
#pragma unroll
        for (int e = 0; e < NC; ++e) {
            const int j = e * 64 + lane;
            if (e < E && j < K)
                L.rbuf[j] = cr[e] - L.v[j];
        }
        lds_sync();
        float w1 = r0, w2 = kLarge;
        int i1 = 0, i2 = -1;
        if (lane == 0) {
            for (int j = 1; j < K; ++j) {
                const float r = L.rbuf[j];
                if (!(r < w2))
                    continue;
                if (r >= w1) {
                    w2 = r;
                    i2 = j;
                } else {
                    w2 = w1;
                    i2 = i1;
                    w1 = r;
                    i1 = j;
                }
            }
        }
        j1 = readlane_i(i1, 0);
        j2 = readlane_i(i2, 0);
        u1 = readlane_f(w1, 0);
        u2 = readlane_f(w2, 0);
        return;
    }
    // first column (in index order) at k1; second: the next one at k1 if
    // k2 == k1, else the first at k2
    // (a key taken from the row always has a column; the guards keep an
    // index in range regardless)
    j1 = first_column<NC>(kk, k1, -1, -1);
    if (j1 == kKeyNone)
        j1 = 0;
    if (k2 != kKeyNone)
        j2 = first_column<NC>(kk, k2, j1, -1);
    if (j2 == kKeyNone)
        j2 = -1;
    u1 = uniform_f(reduced(j1));
    u2 = kLarge;
    if (j2 >= 0) {
        const float w = uniform_f(reduced(j2));
        if (w < kLarge)
            u2 = w;
        else
            j2 = -1;
    }
    if constexpr (LDS::kSlots == 0)
        return;
    if (!refill || j2 < 0)
        return;
    // refill: the third smallest (value, column) after j1, j2 and the fourth
    // smallest value
    int a3 = kKeyNone, b3 = kKeyNone;
#pragma unroll
    for (int e = 0; e < NC; ++e) {
        const int j = e * 64 + lane;
        const int k = (j != j1 && j != j2) ? kk[e] : kKeyNone;
        if (k < a3) {
            b3 = a3;
            a3 = k;
        } else if (k < b3) {
            b3 = k;
        }
    }
    int p3, p4;
    wave_min2_key(a3, p3, p4);
    const int k3 = uniform_i(p3);
    const int k4 = min(uniform_i(p4), uniform_i(wave_min_key(b3)));
    if (k3 == kKeyNone)
        return;
    const int j3 = first_column<NC>(kk, k3, j1, j2);
    if (j3 == kKeyNone)
        return;
    const int lo12 = min(j1, j2), hi12 = max(j1, j2);
    const int s0 = min(lo12, j3), s2 = max(hi12, j3);
    const int s1 = j1 + j2 + j3 - s0 - s2;
    const float g0 = chunk_value(cr, s0 >> 6, s0 & 63);
    const float g1 = chunk_value(cr, s1 >> 6, s1 & 63);
    const float g2 = chunk_value(cr, s2 >> 6, s2 & 63);
    // slots 0..2 by column, the rest empty
    if (lane < kCacheSlots) {
        L.cq[fi][lane] = (int16_t)(lane == 0 ? s0 : (lane == 1 ? s1 : (lane == 2 ? s2 : -1)));
        L.cg[fi][lane] = lane == 0 ? g0 : (lane == 1 ? g1 : g2);
    }
    L.ctau[fi] = k4 == kKeyNone ? finf() : key_to_float(k4);  // every lane, the same word
}

// ---- prefill: the column reduction's minima and every row's cache -----------
//
// Both are many-wave passes over the batch, launched after the statistics
// pass and before the solve when the caller's workspace holds them.  The
// solve then starts its augmenting row reduction with every real row cached
// at depth kCacheSlots: with the duals of the column reduction, which only
// fall afterwards (the reduction transfer and the row reduction lower them),
// so each cache stays valid.  On the slowest problem of a (64, 512, 768)
// batch with 20 % +inf, 745 of its 2,496 row-reduction steps scan their row
// without the prefill and 80 with it.

constexpr int kColminCols = 128;   // columns per block
constexpr int kColminGroups = 8;   // row groups per block: rows g, g + 8, ...
constexpr int kColminRows = 8;     // rows in flight per thread

// The sentinel of the batch from the statistics partials (one wave); false
// when the batch holds NaN / -inf (the solve then writes -1 and nothing of
// the prefill is read).
__device__ __forceinline__ bool prep_sentinel(const JvStats *partial, int n_partial, int K,
                                              float &sentinel) {
    float mx, mn;
    uint32_t flags;
    fold_stats(partial, n_partial, mx, mn, flags);
    sentinel = (flags & kJvFlagAnyFinite) ? (mx + 1.0f) * (float)(K + 1) : 1.0f;
    return !(flags & (kJvFlagNan | kJvFlagNegInf));
}

// v[b][j] = the smallest cost of column j of the padded tile, starting from
// LARGE with row 0 and taking a row only on a strictly smaller cost in row
// order (jonker_dense_flat.h:124-140), y[b][j] = that row: each row group
// folds its rows in order, the groups merge by (cost, row), then the padding
// rows (all 0) win where 0 is strictly smaller.  Grid (B, ceil(K / 128)).
__global__ void __launch_bounds__(kColminCols * kColminGroups)
jv_large_colmin_kernel(const float *__restrict__ costs, int N, int M,
                       const JvStats *__restrict__ partial, int n_partial,
                       float *__restrict__ v_out, int32_t *__restrict__ y_out) {
    const int K = N > M ? N : M;
    const int64_t b = blockIdx.x;
    const int col = (int)(threadIdx.x % kColminCols);
    const int g = (int)(threadIdx.x / kColminCols);
    const int j = (int)blockIdx.y * kColminCols + col;
    float sentinel;
    if (!prep_sentinel(partial, n_partial, K, sentinel))
        return;  // uniform over the block
    float vmin = kLarge;
    int ymin = 0;
    if (j < K) {
        if (j >= M) {
            // a padding column reads 0 in every real row: the group's first row
            if (g < N && 0.f < vmin) {
                vmin = 0.f;
                ymin = g;
            }
        } else {
            const float *src = costs + b * (int64_t)N * M + j;
            for (int i = g; i < N; i += kColminGroups * kColminRows) {
                float c[kColminRows];
#pragma unroll
                for (int u = 0; u < kColminRows; ++u) {
                    const int r = min(i + u * kColminGroups, N - 1);
                    c[u] = src[(int64_t)r * M];
                }
#pragma unroll
                for (int u = 0; u < kColminRows; ++u) {
                    const int r = i + u * kColminGroups;
                    const float cv = isfinite(c[u]) ? c[u] : sentinel;
                    if (r < N && cv < vmin) {
                        vmin = cv;
                        ymin = r;
                    }
                }
            }
        }
    }
    __shared__ float sv[kColminGroups][kColminCols];
    __shared__ int sy[kColminGroups][kColminCols];
    sv[g][col] = vmin;
    sy[g][col] = ymin;
    __syncthreads();
    if (g != 0 || j >= K)
        return;
#pragma unroll
    for (int q = 1; q < kColminGroups; ++q) {
        const float w = sv[q][col];
        const int r = sy[q][col];
        if (w < vmin || (w == vmin && r < ymin)) {
            vmin = w;
            ymin = r;
        }
    }
    if (N < K && 0.f < vmin) {
        vmin = 0.f;
        ymin = N;
    }
    v_out[b * K + j] = vmin;
    y_out[b * K + j] = ymin;
}

// Row i < N of problem b: the kCacheSlots smallest reduced costs c - v
// (v from jv_large_colmin_kernel), in order of (value, column) as the
// reference's scans rank them, stored by ascending column with their costs,
// and tau = the next smallest value.  One wave per row, four per block.
template <int NC>
__global__ void __launch_bounds__(256)
jv_large_rowcache_kernel(const float *__restrict__ costs, int64_t B, int N, int M,
                         const JvStats *__restrict__ partial, int n_partial,
                         const float *__restrict__ v_in, int16_t *__restrict__ cq_out,
                         float *__restrict__ cg_out, float *__restrict__ tau_out) {
    const int K = N > M ? N : M;
    const int E = (K + 63) / 64;
    const int lane = lane_id();
    // each wave's candidates of the threshold selection: keys, columns and
    // costs at fixed offsets from one address
    __shared__ uint32_t rc_cand[4][3][64];
    CostView C;
    C.N = N;
    C.M = M;
    C.sentinel = 1.f;
    bool have_sentinel = false;
    const int64_t rows = B * (int64_t)N;
    // the wave's index is uniform: row bases stay scalar and the loads take
    // a scalar base with 32-bit lane offsets
    const int wave = uniform_i((int)(threadIdx.x >> 6));
    for (int64_t row = (int64_t)blockIdx.x * 4 + wave; row < rows;
         row += (int64_t)gridDim.x * 4) {
        const int64_t b = row / N;
        const int i = (int)(row - b * N);
        C.src = costs + b * (int64_t)N * M;
        const float *vb = v_in + b * K;
        const char *rsrc = reinterpret_cast<const char *>(C.src + (int64_t)i * M);
        const char *vsrc = reinterpret_cast<const char *>(vb);
        // byte offsets from the scalar row bases, clamped into the row; the
        // opaque copy of lane * 4 keeps the compiler from holding all of
        // them (as 64-bit values) across the row loop
        uint32_t lane4 = (uint32_t)lane * 4u;
        asm volatile("" : "+v"(lane4));
        const uint32_t lim_m = (uint32_t)(M - 1) * 4u, lim_k = (uint32_t)(K - 1) * 4u;
        float raw[NC], vv[NC];
#pragma unroll
        for (int e = 0; e < NC; ++e)
            raw[e] = *reinterpret_cast<const float *>(rsrc + min(lane4 + (uint32_t)e * 256u, lim_m));
#pragma unroll
        for (int e = 0; e < NC; ++e)
            vv[e] = *reinterpret_cast<const float *>(vsrc + min(lane4 + (uint32_t)e * 256u, lim_k));
        // the statistics are folded while the row is in flight (the raw
        // costs need the sentinel only from here on)
        if (!have_sentinel) {
            if (!prep_sentinel(partial, n_partial, K, C.sentinel))
                return;
            have_sentinel = true;
        }
        f32x16 cr;
        int kk[NC];
#pragma unroll
        for (int e = 0; e < NC; ++e) {
            const int j = e * 64 + lane;
            // fix_cost in bit operations (its selects became two nested
            // branches per value here): +inf -> sentinel, columns >= M -> 0
            const int rb = __float_as_int(raw[e]);
            const int fin = -(int)((rb & 0x7f800000) != 0x7f800000);
            const int cb = ((rb & fin) | (__float_as_int(C.sentinel) & ~fin)) & -(int)(j < M);
            const float c = __int_as_float(cb);
            cr[e] = c;
            // kKeyNone past the row: the key is formed unconditionally and
            // raised by a max
            kk[e] = max(fkey(c - vv[e]), (e < E && j < K) ? (int)0x80000000 : kKeyNone);
        }
        // Threshold selection.  T = the 17th smallest of the 64 lane minima
        // (as a multiset), from a bitwise search on ballot counts: at least
        // 17 keys are <= T, so the row's 17 smallest (key, column) pairs all
        // are.  The candidates (key <= T; ~20 on the (64, 512, 768) batch)
        // go to LDS in column order, and each takes its rank in (key,
        // column) order from the others: ranks 0..15 are the slots (in
        // column order already), rank 16 gives tau.  More than 64 candidates
        // (wide ties) take the round-by-round selection below.
        {
            uint32_t lmin = 0xffffffffu;
#pragma unroll
            for (int e = 0; e < NC; ++e)
                lmin = min(lmin, (uint32_t)kk[e] ^ 0x80000000u);
            uint32_t T = 0;
#pragma unroll
            for (int bit = 31; bit >= 0; --bit) {
                const uint32_t x = T | ((1u << bit) - 1u);
                const uint64_t m = ballot(lmin <= x);
                if (__builtin_popcount((uint32_t)m) + __builtin_popcount((uint32_t)(m >> 32)) <=
                    kCacheSlots)
                    T |= 1u << bit;
            }
            T = min(T, 0xfffffffeu);  // a missing key (0xffffffff) is never a candidate
            uint32_t *sk = rc_cand[wave][0];
            int *sc = reinterpret_cast<int *>(rc_cand[wave][1]);
            float *sg = reinterpret_cast<float *>(rc_cand[wave][2]);
            int total = 0;
#pragma unroll
            for (int e = 0; e < NC; ++e) {
                const bool cand = ((uint32_t)kk[e] ^ 0x80000000u) <= T;
                const uint64_t m = ballot(cand);
                const int pos = total + lanes_below(m);
                if (cand && pos < 64) {
                    sk[pos] = (uint32_t)kk[e] ^ 0x80000000u;
                    sc[pos] = e * 64 + lane;
                    sg[pos] = cr[e];
                }
                total += __builtin_popcountll(m);
            }
            if (total <= 64) {
                lds_sync();
                const bool have = lane < total;
                const uint32_t mu = have ? sk[lane] : 0xffffffffu;
                const int mc = sc[lane];
                const float mg = sg[lane];
                lds_sync();  // read before the next row's candidates are written
                int rank = 0;
                for (int q = 0; q < total; ++q) {
                    const uint32_t uq = (uint32_t)readlane_i((int)mu, q);
                    rank += (uq < mu || (uq == mu && q < lane)) ? 1 : 0;
                }
                const bool sel = have && rank < kCacheSlots;
                const uint64_t ms = ballot(sel);
                const int nsel = __builtin_popcountll(ms);
                if (sel) {
                    const int slot = lanes_below(ms);
                    cq_out[row * kCacheSlots + slot] = (int16_t)mc;
                    cg_out[row * kCacheSlots + slot] = mg;
                } else if (lane >= nsel && lane < kCacheSlots) {
                    cq_out[row * kCacheSlots + lane] = (int16_t)-1;
                    cg_out[row * kCacheSlots + lane] = 0.f;
                }
                const uint64_t mt = ballot(have && rank == kCacheSlots);
                const float tau =
                    mt == 0 ? finf()
                            : key_to_float((int)((uint32_t)readlane_i((int)mu, first_lane(mt | (1ull << 63))) ^
                                                 0x80000000u));
                if (lane == 0)
                    tau_out[row] = tau;
                continue;
            }
        }
        // Each lane keeps its three smallest (key, chunk) not yet taken, in
        // (key, chunk) order (a later chunk is a larger column).  The row's
        // next smallest (key, column) is then the head of some lane: the
        // smallest key among the heads, and on a tie the smallest column
        // among those heads (the first column at a key is its lane's head).
        // A lane whose three run out while it still holds keys has them
        // rebuilt (with every lane's: the same or longer prefixes).
        int h1, h2, h3, e1, e2, e3;  // keys kKeyNone past the lane's last
        uint32_t taken = 0;
        int n_left = 0;
#pragma unroll
        for (int e = 0; e < NC; ++e)
            n_left += kk[e] != kKeyNone ? 1 : 0;
        auto build = [&]() {
            h1 = h2 = h3 = kKeyNone;
            e1 = e2 = e3 = 0;
#pragma unroll
            for (int e = 0; e < NC; ++e) {
                const int k = (taken >> e) & 1 ? kKeyNone : kk[e];
                const bool l1 = k < h1, l2 = k < h2, l3 = k < h3;
                h3 = l2 ? h2 : (l3 ? k : h3);
                e3 = l2 ? e2 : (l3 ? e : e3);
                h2 = l1 ? h1 : (l2 ? k : h2);
                e2 = l1 ? e1 : (l2 ? e : e2);
                h1 = l1 ? k : h1;
                e1 = l1 ? e : e1;
            }
        };
        build();
        int my_col = -1;
        float my_cost = 0.f;
        int tau_key = kKeyNone;
        for (int t = 0; t <= kCacheSlots; ++t) {
            const int k = wave_min_key_s(h1);
            if (t == kCacheSlots || k == kKeyNone) {
                tau_key = k;
                break;
            }
            const uint64_t m = ballot(h1 == k);
            const int w = (m & (m - 1)) ? (wave_min_key_s(h1 == k ? e1 * 64 + lane : kKeyNone) & 63)
                                        : first_lane(m);
            const int ew = readlane_i(e1, w);
            const float cost = chunk_value(cr, ew, w);
            if (lane == t) {
                my_col = ew * 64 + w;
                my_cost = cost;
            }
            if (lane == w) {
                taken |= 1u << ew;
                --n_left;
                h1 = h2;
                e1 = e2;
                h2 = h3;
                e2 = e3;
                h3 = kKeyNone;
            }
            if (readlane_i(h1, w) == kKeyNone && readlane_i(n_left, w) > 0)
                build();
        }
        // slot = rank of the column among the chosen ones
        int rank = 0;
#pragma unroll
        for (int q = 0; q < kCacheSlots; ++q) {
            const int cq = readlane_i(my_col, q);
            rank += (cq >= 0 && cq < my_col) ? 1 : 0;
        }
        if (lane < kCacheSlots) {
            const int slot = my_col >= 0 ? rank : lane;
            cq_out[row * kCacheSlots + slot] = (int16_t)my_col;
            cg_out[row * kCacheSlots + slot] = my_cost;
        }
        if (lane == 0)
            tau_out[row] = tau_key == kKeyNone ? finf() : key_to_float(tau_key);
    }
}

// COMPACT = false: jonker_dense_flat.h:124-274; COMPACT = true:
// jonker_compact_core.h:51-252 (only called on its value range, where every
// reduced cost stays far below LARGE): the same steps with no cap on the
// augmenting row reduction, the first unassigned column of a minimum group
// ending a path, the dual update (v + d) - min and FLT_MAX as the transfer's
// starting minimum.
template <bool COMPACT, int NC, class LDS>
__device__ __forceinline__ bool large_solve(const int K, const int E, LDS &L, const CostView &C,
                                            const LargePrep &P) {
    const int lane = lane_id();

    // ---- column reduction (ccrrt_dense, jonker_dense_flat.h:124-176) ----
    if (P.v != nullptr) {
        // the minima and their rows from the prefill (jv_large_colmin_kernel)
        float pv[NC];
        int py[NC];
#pragma unroll
        for (int e = 0; e < NC; ++e) {
            const int j = min(e * 64 + lane, K - 1);
            pv[e] = P.v[j];
            py[e] = P.y[j];
        }
#pragma unroll
        for (int e = 0; e < NC; ++e) {
            const int j = min(e * 64 + lane, K - 1);  // past K: column K-1 again
            L.v[j] = pv[e];
            L.y[j] = py[e];
            L.x[j] = -1;   // K rows == K columns
            L.ev[j] = 0;   // claim counts
            L.emap[j] = -1;
        }
    } else {
        float vmin[NC];
        int ymin[NC];
#pragma unroll
        for (int e = 0; e < NC; ++e) {
            vmin[e] = kLarge;
            ymin[e] = 0;
        }
        const int rows_real = C.N < K ? C.N : K;
        // four rows' loads in flight per pass; rows still fold in order
        constexpr int R = 4;
        for (int i = 0; i < rows_real; i += R) {
            float c[R][NC];
#pragma unroll
            for (int q = 0; q < R; ++q)
                load_row_raw<NC>(C, min(i + q, rows_real - 1), c[q]);
#pragma unroll
            for (int q = 0; q < R; ++q)
#pragma unroll
                for (int e = 0; e < NC; ++e) {
                    const int j = e * 64 + lane;
                    const float cv = fix_cost(C, c[q][e], j);
                    if (i + q < rows_real && e < E && j < K && cv < vmin[e]) {
                        vmin[e] = cv;
                        ymin[e] = i + q;
                    }
                }
        }
        // padding rows (all 0): the first one wins where 0 is a strict new minimum
#pragma unroll
        for (int e = 0; e < NC; ++e) {
            const int j = e * 64 + lane;
            if (e < E && j < K) {
                if (rows_real < K && 0.f < vmin[e]) {
                    vmin[e] = 0.f;
                    ymin[e] = rows_real;
                }
                L.v[j] = vmin[e];
                L.y[j] = ymin[e];
                L.x[j] = -1;   // K rows == K columns
                L.ev[j] = 0;   // claim counts
                L.emap[j] = -1;
            }
        }
    }
    lds_sync();
    for (int e = 0; e < E; ++e) {
        const int j = e * 64 + lane;
        if (j < K) {
            atomicMax(&L.x[L.y[j]], j);
            atomicAdd(&L.ev[L.y[j]], 1);
        }
    }
    lds_sync();
    for (int e = 0; e < E; ++e) {
        const int j = e * 64 + lane;
        if (j < K && L.x[L.y[j]] != j)
            L.y[j] = -1;
    }
    lds_sync();
    // free rows in increasing order, then reduction transfer for unique rows
    int n_free = 0;
    for (int e = 0; e < E; ++e) {
        const int i = e * 64 + lane;
        const bool fre = i < K && L.x[i] < 0;
        const uint64_t m = ballot(fre);
        const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
        if (fre)
            L.fr[n_free + __builtin_popcountll(m & below)] = i;
        n_free += __builtin_popcountll(m);
    }
    lds_sync();
    for (int e = 0; e < E; ++e) {
        uint64_t t = ballot(e * 64 + lane < K && L.x[e * 64 + lane] >= 0 &&
                            L.ev[e * 64 + lane] <= 1);
        while (t) {
            const int i = e * 64 + first_lane(t);
            t &= t - 1;
            const int own = L.x[i];
            // mn = LARGE, then `if (c < mn) mn = c` over j != own in order
            float cr[NC];
            load_row<NC>(C, i, cr);
            int best = kKeyNone;
            float vv[NC];
#pragma unroll
            for (int e2 = 0; e2 < NC; ++e2)
                vv[e2] = L.v[min(e2 * 64 + lane, K - 1)];
#pragma unroll
            for (int e2 = 0; e2 < NC; ++e2) {
                const int j = e2 * 64 + lane;
                if (e2 < E && j < K) {
                    const float r = j != own ? cr[e2] - vv[e2] : finf();
                    L.rbuf[j] = r;
                    if (j != own)
                        best = min(best, fkey(r));
                }
            }
            best = uniform_i(wave_min_key(best));
            lds_sync();
            const float start_min = COMPACT ? kFltMax : kLarge;
            float mn = start_min;
            if (best < fkey(start_min)) {
                for (int e2 = 0; e2 < E; ++e2) {
                    const int j = e2 * 64 + lane;
                    const uint64_t hit = ballot(j < K && j != own && fkey(L.rbuf[j]) == best);
                    if (hit) {
                        mn = L.rbuf[e2 * 64 + first_lane(hit)];
                        break;
                    }
                }
            }
            if (lane == 0)
                L.v[own] -= mn;
            lds_sync();
        }
    }

    // ---- augmenting row reduction (carr_dense, jonker_dense_flat.h:178-235) ----
    const uint32_t rr_limit =
        COMPACT ? compact_arr_guard(K) : 4u * (uint32_t)K * (uint32_t)K + 64u;
    constexpr bool kCache = LDS::kSlots > 0;  // K > kMaxLargeK: every step scans
    if constexpr (!kCache) {
    } else if (P.v != nullptr) {
        // every real row's cache from the prefill (jv_large_rowcache_kernel)
        copy_to_lds(&L.cq[0][0], P.cq, C.N * kCacheSlots / 2);  // dwords of 16-bit columns
        copy_to_lds(&L.cg[0][0], P.cg, C.N * kCacheSlots);
        float t[NC];
#pragma unroll
        for (int e = 0; e < NC; ++e)
            t[e] = P.ctau[min(e * 64 + lane, C.N - 1)];
#pragma unroll
        for (int e = 0; e < NC; ++e) {
            const int i = min(e * 64 + lane, K - 1);
            L.ctau[i] = i < C.N ? t[e] : -finf();
        }
    } else {
        for (int i = lane; i < K; i += 64)
            L.ctau[i] = -finf();
        // Every slot empty (column -1): the hit tests below compare keys of
        // the slots' costs, and a stale LDS word read as a cost could be a
        // NaN whose key is below tau's even at tau = -inf.
        int32_t *cq32 = reinterpret_cast<int32_t *>(&L.cq[0][0]);
        for (int w = lane; w < C.N * (kCacheSlots / 2); w += 64)
            cq32[w] = -1;
    }
    lds_sync();
    // lanes 0..kCacheSlots-1 hold the cache slots: a slot column is live
    // when below this bound (K there, 0 in the other lanes)
    const uint32_t slot_bound = lane < kCacheSlots ? (uint32_t)K : 0u;
    // Rows >= N of the padded tile are all 0, so their reduced costs are -v:
    // one two-minimum serves every such row until a dual changes (their
    // minima tie too often for the cache's strict tau test).
    int pad_j1 = -1, pad_j2 = -1;
    float pad_u1 = 0.f, pad_u2 = 0.f;
    bool pad_valid = false;
    for (int round = 0; n_free > 0 && round < 2; ++round) {
        uint32_t cur = 0, rr = 0;
        int still = 0;
        // The row of the next step is known before this step ends: the row
        // this step displaces when it lowers a dual (it goes back to the
        // queue's head), else the queue entry after this row.  A step writes
        // the queue only at positions < cur (the slot it consumed, or still
        // <= that slot), so that entry is read at the step's start and its
        // load overlaps the step.  The next row's cache slots (tau, columns,
        // costs) then load as soon as that row is known: after this step's
        // scan refills a cache row, before its other writes (which touch no
        // cache word).
        int fi_next = uniform_i(L.fr[0]);
        float tau_n = 0.f, g_n = 0.f;
        int q_n = 0;
        if constexpr (kCache) {
            tau_n = L.ctau[fi_next];
            q_n = L.cq[fi_next][lane & (kCacheSlots - 1)];
            g_n = L.cg[fi_next][lane & (kCacheSlots - 1)];
        }
        // The end of a step (carr_dense's update, jonker_dense_flat.h:
        // 210-232), given row fi's two minima j1 / j2 (j2 = -1: none), their
        // owners y1 / y2, v[j1], lowered = v[j1] - (u2 - u1) and whether it
        // is below v[j1] (lowers, 0 / 1).  Flags as 0 / 1 integers keep the
        // logic on the scalar unit.  x is not written here: it is rebuilt
        // from y after the reduction (no step reads it).
        // (x >> 31) & 1 for "x < 0": a compare's flag would be kept as a
        // lane mask, and turned into 0 / 1 on the vector unit.
        auto neg = [](int x) { return (int)((uint32_t)x >> 31); };
        auto finish = [&](int fi, int fqs, int j1, int j2, int y1, int y2, float vj1, float lowered,
                          int lowers) __attribute__((always_inline)) {
            // rr and cur * K stay below 2^31 (rr_limit)
            const int cap = COMPACT ? 1 : neg((int)(rr - cur * (uint32_t)K));
            // dec: v[j1] falls and the displaced row goes back to the queue's
            // head; sw: no fall, the row takes j2 when j1 is owned
            const int dec = cap & lowers;
            const int sw = cap & (lowers ^ 1) & (neg(y1) ^ 1) & (neg(j2) ^ 1);
            const int jsel = sw ? j2 : j1;
            const int i0 = sw ? y2 : y1;
            const int push = neg(i0) ^ 1;
            const int back = dec & push;  // the displaced row is the next row
            const int tail = push & (dec ^ 1);  // ... or it joins the next round
            const uint32_t slot = cur - 1;  // the queue slot this step consumed
            fi_next = back ? i0 : fqs;
            if constexpr (kCache) {
                // clamped: after the last step fq is read past the queue
                const int rn = min(max(fi_next, 0), K - 1);
                tau_n = L.ctau[rn];
                q_n = L.cq[rn][lane & (kCacheSlots - 1)];
                g_n = L.cg[rn][lane & (kCacheSlots - 1)];
            }
            lds_sync();
            // Every write unconditional, every lane writing the same word:
            // v[j1] gets its own value back when it does not fall, and a row
            // that displaces no one writes -1 into the consumed slot, which
            // is dead (the next round's rows sit below it: still <= slot).
            L.v[j1] = __int_as_float(dec ? __float_as_int(lowered) : __float_as_int(vj1));
            L.fr[tail ? (uint32_t)still : slot] = i0;
            L.y[jsel] = fi;
            pad_valid = pad_valid && !dec;
            cur -= back;
            still += tail;
            lds_sync();
        };
        // The step loop's speed moves by up to 2.5 % with its offset in the
        // 64-byte instruction-cache line (C3 batch 1.030-1.055 ms over the
        // offsets 0-7, each a few nops from the line's start); pinned at a
        // fast one so that edits elsewhere in the kernel do not move it.
        asm volatile(".p2align 6\n\ts_nop 0\n\ts_nop 0" ::: "memory");
        while (cur < (uint32_t)n_free) {
            ++rr;
            if (rr > rr_limit)
                return false;
            // LDS words every lane reads alike are made uniform explicitly, so
            // that the step's branches are scalar (no exec-mask bookkeeping)
            const int fi = fi_next;
            ++cur;
            const int fq = L.fr[min(cur, (uint32_t)K - 1)];
            if (kCache && fi < C.N) {
                // The cached two minima, straight-line to the step's end.
                // No branch on tau: a row never filled has tau = -inf and
                // every slot empty.  Slot columns outside [0, K) read column
                // 0 and carry no key.  tau as a key: fkey is monotone and tau was stored
                // from a key, so u2 < tau <=> key(u2) < key(tau); and u2 <
                // LARGE, so that the reference's (LARGE, -1) start slot
                // cannot win.
                const int tb = uniform_i(__float_as_int(tau_n));
                const int ktau = min(tb ^ ((tb >> 31) & 0x7fffffff), kKeyLarge);
                const bool qok = (uint32_t)q_n < slot_bound;
                const int q = qok ? q_n : 0;
                const float vq = L.v[q];
                const int yq = L.y[q];
                const float r = g_n - vq;
                // the owners are needed only by a cache hit, but their load
                // is kept beside the duals' (the compiler would otherwise
                // sink it into the hit's branch, a third round trip)
                asm volatile("" ::"v"(yq));
                // lane s < kCacheSlots holds slot s (columns ascending with
                // the slot): the first lane at a key is the first column at
                // that key
                const int key = qok ? fkey(r) : kKeyNone;
                int p1, p2;
                min2_16_key(key, p1, p2);
                const int k1 = readlane_i(p1, 0), k2 = readlane_i(p2, 0);
                const int fqs = uniform_i(fq);
                // the two ballots issue together (k1 <= k2, and kKeyNone is
                // above every key)
                const uint64_t m1 = ballot(key == k1), m2 = ballot(key == k2);
                if (k2 < ktau) {
                    // u1, u2 from the keys (lanes 0..15 hold both), beside
                    // the lane search: the keys fold -0.0 into +0.0, which
                    // changes u2 - u1 only when both are zeros, and then
                    // lowered is a zero that is not below v[j1] and is not
                    // stored.  Every lane lowers its own slot's dual; lane
                    // l1's is the step's.
                    const float low = vq - (key_to_float(p2) - key_to_float(p1));
                    const uint64_t mlow = ballot(low < vq);
                    const int pk = (yq << 16) | q;  // q < K <= 1024, yq in [-1, K)
                    const int l1 = first_lane(m1);
                    const int l2 = first_lane(m2 & ~(1ull << l1));
                    const int pk1 = readlane_i(pk, l1), pk2 = readlane_i(pk, l2);
                    finish(fi, fqs, pk1 & 0xffff, pk2 & 0xffff, pk1 >> 16, pk2 >> 16, readlane_f(vq, l1),
                           readlane_f(low, l1), (int)(mlow >> l1) & 1);
                    continue;
                }
            }
            // a padded row, or a cache miss: the row's scan (which refills
            // a real row's cache)
            const bool pad_row = fi >= C.N;
            if (pad_row && pad_valid && pad_j2 >= 0) {
                // A run of padded rows while no dual falls.  Each of them
                // has the same two minima (j1, j2) and lowers nothing, so
                // step by step: the first takes j1 when j1 is free, every
                // later one takes j2 and pushes j2's previous owner to the
                // next round's list (still), and the next row is the next
                // queue entry.  The run -- this row and the padded rows
                // queued after it, within the step budget -- is done at
                // once: the pushed rows are y[j2] (when owned) and the
                // j2-takers but the last, copied 64 at a time, then the two
                // owners.  The copy's target never passes its source by
                // more than one entry (still <= the consumed slot), and each
                // window is written only after the next one is read.
                const float vj1 = uniform_f(L.v[pad_j1]);
                const int cap = COMPACT ? 1 : neg((int)(rr - cur * (uint32_t)K));
                if (cap && !(vj1 - (pad_u2 - pad_u1) < vj1)) {
                    const uint32_t first = cur - 1;  // this row's slot
                    const uint32_t budget = rr_limit - rr;  // further steps allowed
                    uint32_t R = 1;
                    for (uint32_t base = cur; R - 1 < budget; base += 64) {
                        const uint32_t p = base + lane;
                        const int r = L.fr[min(p, (uint32_t)K - 1)];
                        const uint64_t pm = ballot(p < (uint32_t)n_free && r >= C.N);
                        const uint32_t lead = ~pm == 0 ? 64u : (uint32_t)__builtin_ctzll(~pm);
                        R += lead;
                        if (lead < 64)
                            break;
                    }
                    R = min(R, budget + 1);
                    const int y1 = uniform_i(L.y[pad_j1]);
                    const int y2 = uniform_i(L.y[pad_j2]);
                    const uint32_t s0 = y1 < 0 ? 1u : 0u;  // the first row takes j1
                    const int last = uniform_i(L.fr[first + R - 1]);
                    if (R > s0) {
                        const uint32_t src0 = first + s0, n_copy = R - 1 - s0;
                        const uint32_t dst0 = (uint32_t)still + (y2 >= 0 ? 1u : 0u);
                        int nxt = L.fr[min(src0 + lane, (uint32_t)K - 1)];
                        for (uint32_t w = 0; w < n_copy; w += 64) {
                            const int val = nxt;
                            nxt = L.fr[min(src0 + w + 64 + lane, (uint32_t)K - 1)];
                            lds_sync();
                            if (w + lane < n_copy)
                                L.fr[dst0 + w + lane] = val;
                            lds_sync();
                        }
                        if (y2 >= 0)
                            L.fr[still] = y2;  // every lane writes the same word
                        L.y[pad_j2] = last;
                        still += (int)n_copy + (y2 >= 0 ? 1 : 0);
                    }
                    if (s0)
                        L.y[pad_j1] = fi;
                    rr += R - 1;
                    cur += R - 1;
                    lds_sync();
                    fi_next = uniform_i(L.fr[min(cur, (uint32_t)K - 1)]);
                    if constexpr (kCache) {
                        const int rn = min(max(fi_next, 0), K - 1);
                        tau_n = L.ctau[rn];
                        q_n = L.cq[rn][lane & (kCacheSlots - 1)];
                        g_n = L.cg[rn][lane & (kCacheSlots - 1)];
                    }
                    continue;
                }
            }
            int j1, j2;
            float u1, u2;
            if (pad_row && pad_valid) {
                j1 = pad_j1;
                j2 = pad_j2;
                u1 = pad_u1;
                u2 = pad_u2;
            } else {
                scan_row<NC>(L, C, fi, E, K, !pad_row, j1, j2, u1, u2);
                if (pad_row) {
                    pad_j1 = j1;
                    pad_j2 = j2;
                    pad_u1 = u1;
                    pad_u2 = u2;
                    pad_valid = true;
                }
            }
            const float vj1 = uniform_f(L.v[j1]);
            const float lowered = vj1 - (u2 - u1);
            finish(fi, uniform_i(fq), j1, j2, uniform_i(L.y[j1]), uniform_i(L.y[max(j2, 0)]), vj1,
                   lowered, lowered < vj1 ? 1 : 0);
        }
        n_free = still;
    }
    // x from y (the row-reduction steps write y alone)
    for (int i = lane; i < K; i += 64)
        L.x[i] = -1;
    lds_sync();
    for (int j = lane; j < K; j += 64) {
        const int i = L.y[j];
        if (i >= 0)
            L.x[i] = j;
    }
    lds_sync();

    // ---- augmentation (ca_dense / find_path_dense, jonker_dense_flat.h:75-122,237-258) ----
    // A run of padded start rows: their rows are all 0, so while no dual
    // changes the first find_dense of each sees the same tied block (the
    // columns at the largest v), and each path takes the next unassigned
    // column of it.  The run's first path lists the block's unassigned
    // columns in pick order (dense: descending, compact: ascending) in
    // rbuf, unused by the paths; later padded paths take the next entry
    // still unassigned (a real row's single-column path may have taken
    // one).  A full search, which moves duals, ends the run.
    // Each padded start scans the list from run_pos and takes the first
    // entry still unassigned, so a run of consecutive padded starts takes
    // the list's unassigned entries in order: the k-th start of the run the
    // k-th.  That is done 64 starts against 64 entries per round (ranks
    // from a ballot); run_pos then stands where the sequential scans would
    // leave it: after the last entry taken, or past the window when the
    // starts outnumber its unassigned entries.  A start the list cannot
    // serve (it ran out) or a real row takes the paths below.
    int *const run_list = reinterpret_cast<int *>(L.rbuf);
    int run_pos = 0, run_n = 0;
    for (int f = 0; f < n_free; ++f) {
        int start = uniform_i(L.fr[f]);
        if (start >= C.N && run_pos < run_n) {
            do {
                const int fl = f + lane;
                const int sl = L.fr[min(fl, K - 1)];
                const uint64_t padm = ballot(fl < n_free && sl >= C.N);
                const int R = ~padm == 0 ? 64 : (int)__builtin_ctzll(~padm);  // >= 1
                const int pl = run_pos + lane;
                const int el = run_list[min(pl, run_n - 1)];
                const bool opn = pl < run_n && L.y[el] < 0;
                const uint64_t om = ballot(opn);
                const int A = min(R, (int)__builtin_popcountll(om));
                const int k = lanes_below(om);  // rank of an open entry
                const int sk = __shfl(sl, min(k, 63));  // its start row
                if (opn && k < A) {
                    L.y[el] = sk;
                    L.x[sk] = el;
                }
                if (A == R)  // every start served: after the A-th open entry
                    run_pos += first_lane(ballot(opn && k == A - 1)) + 1;
                else  // the window's unassigned entries all taken, the rest skipped
                    run_pos = min(run_pos + 64, run_n);
                f += A;
                lds_sync();
            } while (f < n_free && run_pos < run_n && uniform_i(L.fr[f]) >= C.N);
            if (f >= n_free)
                break;
            start = uniform_i(L.fr[f]);
        }
        // The first find_dense from the start row's cache, without its row:
        // when the smallest cached reduced cost is below tau, it is the
        // row's minimum and every column tied with it is cached (all others
        // are >= tau: duals only fall, in the row reduction and in the
        // path updates below alike).  Its tied block in column order is
        // then the cached columns at that key (slots ascend with the
        // column), and when one of them is unassigned the path is that
        // single column, as below.
        if (kCache && start < C.N) {
            const float tau_l = L.ctau[start];
            const int qs = L.cq[start][lane & (kCacheSlots - 1)];
            const float g = L.cg[start][lane & (kCacheSlots - 1)];
            __builtin_amdgcn_sched_barrier(0);
            const int tb = uniform_i(__float_as_int(tau_l));
            const int ktau = tb ^ ((tb >> 31) & 0x7fffffff);
            const bool qok = (uint32_t)qs < slot_bound;
            const int q = qok ? qs : 0;
            const float vq = L.v[q];
            const int yq = L.y[q];
            const int key = qok ? fkey(g - vq) : kKeyNone;
            const int mk = wave_min_key_s(key);
            if (mk < ktau) {
                const uint64_t open = ballot(key == mk && yq < 0);
                if (open) {
                    const int found = readlane_i(q, COMPACT ? first_lane(open) : last_lane(open));
                    L.y[found] = start;  // every lane writes the same word
                    L.x[start] = found;
                    lds_sync();
                    continue;
                }
            }
        }
        float cr[NC];
        load_row<NC>(C, start, cr);
        // The first find_dense, decided from the row in registers: cols[] is
        // the identity, so its tied block is, in column order, every column
        // whose d = c - v has the row's minimum key (the column of the last
        // new running minimum is the first of them, the ties after it the
        // rest).  When one of them is unassigned the path is that single
        // column -- dense takes the last such column, compact the first --
        // and neither cols / d / pred nor the event list is needed.
        {
            // duals and owners read outside any guard, all in flight together
            int dk[NC], yv[NC];
            float vv[NC];
#pragma unroll
            for (int e = 0; e < NC; ++e) {
                vv[e] = L.v[min(e * 64 + lane, K - 1)];
                yv[e] = L.y[min(e * 64 + lane, K - 1)];
            }
            int mk = kKeyNone;
#pragma unroll
            for (int e = 0; e < NC; ++e) {
                const int j = e * 64 + lane;
                dk[e] = (e < E && j < K) ? fkey(cr[e] - vv[e]) : kKeyNone;
                mk = min(mk, dk[e]);
            }
            mk = wave_min_key_s(mk);
            int found = -1;
            uint64_t open[NC];
#pragma unroll
            for (int e = 0; e < NC; ++e) {
                open[e] = ballot((dk[e] == mk) & (yv[e] < 0));
                if (COMPACT) {
                    if (open[e] && found < 0)
                        found = e * 64 + first_lane(open[e]);
                } else if (open[e]) {
                    found = e * 64 + last_lane(open[e]);
                }
            }
            if (found >= 0) {
                if (start >= C.N) {
                    // the run's list; its first entry is found
                    int n = 0;
#pragma unroll
                    for (int t = 0; t < NC; ++t) {
                        const int e = COMPACT ? t : NC - 1 - t;
                        const uint64_t m = open[e];
                        const uint64_t below = m & ((1ull << lane) - 1);
                        const int rank = COMPACT ? __popcll(below) : __popcll(m) - 1 - __popcll(below);
                        if ((m >> lane) & 1)
                            run_list[n + rank] = e * 64 + lane;
                        n += __popcll(m);
                    }
                    run_pos = 1;
                    run_n = n;
                }
                L.y[found] = start;  // every lane writes the same word
                L.x[start] = found;
                lds_sync();
                continue;
            }
        }
        run_n = 0;  // the full search below moves duals
        float vv[NC];  // read outside the guard, all in flight together
#pragma unroll
        for (int e = 0; e < NC; ++e)
            vv[e] = L.v[min(e * 64 + lane, K - 1)];
#pragma unroll
        for (int e = 0; e < NC; ++e) {
            const int j = e * 64 + lane;
            if (e < E && j < K) {
                L.cols[j] = j;
                L.d[j] = cr[e] - vv[e];
                L.pred[j] = start;
            }
        }
        lds_sync();
        int lo = 0, hi = 0, n_ready = 0, final_j = -1;

        float group_level = 0.f;  // d of the current minimum group
        while (final_j < 0) {
            if (lo >= K)
                return false;
            if (lo == hi) {
                // find_dense over positions [lo, K): classify each position
                // against the running minimum of the positions before it
                n_ready = lo;
                // the next chunk's key is read while this chunk is classified
                auto chunk_key = [&](int base) {
                    const int p = base + lane;
                    const float dv = L.d[L.cols[min(p, K - 1)]];
                    return p < K ? fkey(dv) : kKeyNone;
                };
                int carry = kKeyNone;
                int n_ev = 0;
                int dk_next = chunk_key(lo);
#pragma unroll 1
                for (int base = lo; base < K; base += 64) {
                    const int p = base + lane;
                    const int dk = dk_next;
                    dk_next = chunk_key(base + 64);
                    const int incl = wave_prefix_min_key(dk);
                    const int before = min(carry, wave_shift_up_key(incl));
                    const bool later = p > lo && p < K;
                    const uint64_t rec = ballot(later && dk < before);
                    const uint64_t tie = ballot(later && dk == before);
                    const uint64_t evm = rec | tie;
                    n_ev = append_events(L, n_ev, evm, base, 0x80000000u, rec);
                    carry = min(carry, readlane_i(incl, 63));
                }
                lds_sync();
                hi = replay_find_events(L, n_ev, lo);
                group_level = L.d[L.cols[lo]];
                // dense: the LAST unassigned column of the tied block wins
                // (jonker_dense_flat.h:96-103); compact: the first
                // (jonker_compact_core.h:200-206)
                int pick = -1;
                for (int base = lo; base < hi; base += 64) {
                    const int p = base + lane;
                    const uint64_t open = ballot(p < hi && L.y[L.cols[p]] < 0);
                    if (open) {
                        pick = base + (COMPACT ? first_lane(open) : last_lane(open));
                        if (COMPACT)
                            break;
                    }
                }
                if (pick >= 0)
                    final_j = L.cols[pick];
            }
            if (final_j >= 0)
                break;
            // scan_dense
            int slo = lo, shi = hi;
            bool early = false;
            while (slo != shi) {
                const int q = slo++;
                const int jq = L.cols[q];
                const int iq = L.y[jq];
                // the group's common d: compact uses the level of its
                // gathering, dense the scanned column's own d (equal values)
                const float level = COMPACT ? group_level : L.d[jq];
                int n_ev = 0;
                const int base0 = shi;
                // gather row iq at column jq and at the columns of positions
                // [shi, K), all loads in flight together
                int jg[NC];
                float cg[NC];
#pragma unroll
                for (int e = 0; e < NC; ++e) {
                    const int p = base0 + e * 64 + lane;
                    const int cp = L.cols[min(p, K - 1)];  // outside the guard
                    jg[e] = p < K ? cp : 0;
                }
                float cq = 0.f;
                if (iq < C.N) {
                    const float *srow = C.src + (int64_t)iq * C.M;
                    cq = srow[min(jq, C.M - 1)];
#pragma unroll
                    for (int e = 0; e < NC; ++e)
                        cg[e] = srow[min(jg[e], C.M - 1)];
                    cq = fix_cost(C, cq, jq);
#pragma unroll
                    for (int e = 0; e < NC; ++e)
                        cg[e] = fix_cost(C, cg[e], jg[e]);
                } else {
#pragma unroll
                    for (int e = 0; e < NC; ++e)
                        cg[e] = 0.f;
                }
                const float hq = cq - L.v[jq] - level;
#pragma unroll
                for (int e = 0; e < NC; ++e) {
                    const int base = base0 + e * 64;
                    if (base >= K)
                        break;
                    const int p = base + lane;
                    // jg[e] is a column for every lane (0 past K)
                    const int jp = p < K ? jg[e] : 0;
                    const float vj = L.v[jp], dj = L.d[jp];
                    const int yj = L.y[jp];
                    const float r = p < K ? cg[e] - vj - hq : 0.f;
                    const float dp = p < K ? dj : 0.f;
                    const bool better = p < K && r < dp;
                    const bool tie = better && r == level;
                    const uint64_t ret = ballot(tie & (yj < 0));
                    if (ret) {
                        const int kk = first_lane(ret);
                        // compact stops before relaxing column kk itself
                        if (better && (COMPACT ? lane < kk : lane <= kk))
                            L.d[jp] = r;
                        if (better && lane <= kk)
                            L.pred[jp] = iq;
                        final_j = readlane_i(jp, kk);
                        early = true;
                        break;
                    }
                    if (better) {
                        L.d[jp] = r;
                        L.pred[jp] = iq;
                    }
                    n_ev = append_events(L, n_ev, ballot(tie), base, 0u, 0ull);
                }
                lds_sync();
                if (early)
                    break;
                if (n_ev > 0)
                    apply_tie_run(L, 0, n_ev, shi);
                shi += n_ev;
            }
            if (!early) {
                lo = slo;
                hi = shi;
            }
        }
        const float level = L.d[L.cols[lo]];
        for (int base = 0; base < n_ready; base += 64) {
            const int p = base + lane;
            if (p < n_ready) {
                const int j = L.cols[p];
                L.v[j] = COMPACT ? (L.v[j] + L.d[j]) - level : L.v[j] + (L.d[j] - level);
            }
        }
        lds_sync();
        if (lane == 0) {
            int j = final_j, i;
            int steps = 0;
            do {
                i = L.pred[j];
                L.y[j] = i;
                const int prev = L.x[i];
                L.x[i] = j;
                j = prev;
                if (++steps >= K)
                    break;
            } while (i != start);
        }
        lds_sync();
    }
    return true;
}

template <bool COMPACT, int NC>
__global__ void __launch_bounds__(64)
jv_solve_large_kernel(const float *__restrict__ costs, int64_t B, int N, int M,
                      const JvStats *__restrict__ partial, int n_partial, LargePrep prep,
                      int64_t *__restrict__ out, uint32_t *__restrict__ status) {
    // past 16 chunks (K > 1024) the cache-less layout
    __shared__ typename std::conditional<(NC > kMaxChunks), LargeLdsXL, LargeLds>::type L;
    const int lane = lane_id();
    const int K = N > M ? N : M;
    const int E = (K + 63) / 64;
    const int64_t b = blockIdx.x;
    float mx, mn;
    uint32_t flags;
    fold_stats(partial, n_partial, mx, mn, flags);
    if (b == 0 && lane == 0)
        status[0] = flags;
    int64_t *ob = out + b * N;
    if (flags & (kJvFlagNan | kJvFlagNegInf)) {
        for (int i = lane; i < N; i += 64)
            ob[i] = -1;
        return;
    }
    const bool any_finite = (flags & kJvFlagAnyFinite) != 0;
    CostView C;
    C.src = costs + b * (int64_t)N * M;
    C.N = N;
    C.M = M;
    C.sentinel = any_finite ? (mx + 1.0f) * (float)(K + 1) : 1.0f;
    bool ok;
    if (!COMPACT || compact_wave_range(any_finite, mx, mn, (flags & kJvFlagPosInf) != 0,
                                       C.sentinel)) {
        LargePrep P{nullptr, nullptr, nullptr, nullptr, nullptr};
        if (prep.v != nullptr) {
            P.v = prep.v + b * K;
            P.y = prep.y + b * K;
            P.cq = prep.cq + b * N * kCacheSlots;
            P.cg = prep.cg + b * N * kCacheSlots;
            P.ctau = prep.ctau + b * N;
        }
        ok = large_solve<COMPACT, NC>(K, E, L, C, P);
    } else {
        // compact outside the wave path's range: the lane-serial transcription
        if (lane == 0) {
            auto cost = [C](int i, int j) {
                return (i >= C.N || j >= C.M) ? 0.f : fix_cost(C, C.src[(int64_t)i * C.M + j], j);
            };
            L.ev[0] = compact_serial((uint32_t)K, cost, L.x, L.y, L.fr, L.pred, L.cols, L.v,
                                     L.d) ? 1 : 0;
        }
        lds_sync();
        ok = L.ev[0] != 0;
    }
    if (!ok) {
        if (lane == 0)
            raise_guard(status);
        for (int i = lane; i < N; i += 64)
            ob[i] = -1;
        return;
    }
    for (int i = lane; i < N; i += 64) {
        const int j = L.x[i];
        ob[i] = (j >= 0 && j < M) ? (int64_t)j : (int64_t)-1;
    }
}

} // namespace

namespace {
size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// The prefill's arrays in a workspace of jv_large_prep_bytes(B, N, M).
struct PrepBuffers {
    float *v;
    int32_t *y;
    int16_t *cq;
    float *cg;
    float *ctau;
};

PrepBuffers prep_buffers(void *ws, int64_t B, int N, int M) {
    const int64_t K = N > M ? N : M;
    char *p = static_cast<char *>(ws);
    PrepBuffers r;
    r.v = reinterpret_cast<float *>(p);
    p += align256((size_t)(B * K) * 4);
    r.y = reinterpret_cast<int32_t *>(p);
    p += align256((size_t)(B * K) * 4);
    r.cq = reinterpret_cast<int16_t *>(p);
    p += align256((size_t)(B * N) * kCacheSlots * 2);
    r.cg = reinterpret_cast<float *>(p);
    p += align256((size_t)(B * N) * kCacheSlots * 4);
    r.ctau = reinterpret_cast<float *>(p);
    return r;
}

// One instantiation per chunk count (64-column chunks per lane: K <= 128,
// 256, 512, 768, 1024), so the per-lane loops run over the chunks a row has.
// With a prefill workspace the column minima and the row caches are built
// by two many-wave launches first.
template <bool COMPACT>
int launch_large(const float *costs, int64_t B, int N, int M, const JvStats *partial,
                 int n_partial, void *prep_ws, int64_t *out, uint32_t *status,
                 hipStream_t stream) {
    const int K = N > M ? N : M;
    const int E = (K + 63) / 64;
    LargePrep prep{nullptr, nullptr, nullptr, nullptr, nullptr};
    if (prep_ws != nullptr && K <= kMaxLargeK) {
        const PrepBuffers pb = prep_buffers(prep_ws, B, N, M);
        hipLaunchKernelGGL(jv_large_colmin_kernel,
                           dim3((unsigned)B, (unsigned)((K + kColminCols - 1) / kColminCols)),
                           dim3(kColminCols * kColminGroups), 0, stream, costs, N, M, partial,
                           n_partial, pb.v, pb.y);
        if (hipGetLastError() != hipSuccess)
            return kTmErrLaunch;
        const int64_t rows = B * (int64_t)N;
        const int64_t want = (rows + 3) / 4;
        const unsigned grid = (unsigned)(want < 65536 ? want : 65536);
        auto fill = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, dim3(grid), dim3(256), 0, stream, costs, B, N, M, partial,
                               n_partial, pb.v, pb.cq, pb.cg, pb.ctau);
            return hipGetLastError() == hipSuccess;
        };
        const bool ok = E <= 2    ? fill(jv_large_rowcache_kernel<2>)
                        : E <= 4  ? fill(jv_large_rowcache_kernel<4>)
                        : E <= 8  ? fill(jv_large_rowcache_kernel<8>)
                        : E <= 12 ? fill(jv_large_rowcache_kernel<12>)
                                  : fill(jv_large_rowcache_kernel<kMaxChunks>);
        if (!ok)
            return kTmErrLaunch;
        prep = LargePrep{pb.v, pb.y, pb.cq, pb.cg, pb.ctau};
    }
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3((unsigned)B), dim3(64), 0, stream, costs, B, N, M,
                           partial, n_partial, prep, out, status);
        return hipGetLastError() == hipSuccess ? kTmOk : kTmErrLaunch;
    };
    if (E <= 2)
        return go(jv_solve_large_kernel<COMPACT, 2>);
    if (E <= 4)
        return go(jv_solve_large_kernel<COMPACT, 4>);
    if (E <= 8)
        return go(jv_solve_large_kernel<COMPACT, 8>);
    if (E <= 12)
        return go(jv_solve_large_kernel<COMPACT, 12>);
    if (E <= kMaxChunks)
        return go(jv_solve_large_kernel<COMPACT, kMaxChunks>);
    return go(jv_solve_large_kernel<COMPACT, kXLChunks>);
}
} // namespace

size_t jv_large_prep_bytes(int64_t B, int N, int M) {
    const int64_t K = N > M ? N : M;
    if (K > kMaxLargeK)
        return 0;  // no prefill past the cached layout
    return 2 * align256((size_t)(B * K) * 4) + align256((size_t)(B * N) * kCacheSlots * 2) +
           align256((size_t)(B * N) * kCacheSlots * 4) + align256((size_t)(B * N) * 4);
}

int launch_jv_large(const float *costs, int64_t B, int N, int M, const JvStats *partial,
                    int n_partial, void *prep_ws, int64_t *out, uint32_t *status,
                    hipStream_t stream) {
    return launch_large<false>(costs, B, N, M, partial, n_partial, prep_ws, out, status, stream);
}

int launch_jv_compact_large(const float *costs, int64_t B, int N, int M,
                            const JvStats *partial, int n_partial, void *prep_ws, int64_t *out,
                            uint32_t *status, hipStream_t stream) {
    return launch_large<true>(costs, B, N, M, partial, n_partial, prep_ws, out, status, stream);
}

int jv_large_max_k() { return kMaxXLK; }

int jv_compact_max_k() { return kMaxXLK; }

} // namespace tmamd
