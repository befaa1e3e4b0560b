// jv_compact_large.hip -- assignment::jonker_compact_batch for 64 < K <= 1024
// (gfx950).
//
// Same contract as the K <= 64 compact kernel in jv_batch.hip: the int64
// row->col mapping of torchmatch's CPU op bit for bit
// (sources/torchmatch/assignment/cpu/ops.cpp:176-289,431-433 around
//  sources/torchmatch/assignment/cpu/jonker_compact_core.h:20-252; the
// compact rules are listed in jv_compact.h).
//
// One 64-lane workgroup per problem.  The K x K tile does not fit in LDS, so
// costs are read from global memory (L2 / Infinity Cache) through a view that
// pads virtually (rows >= N and columns >= M read 0) and maps non-finite
// costs to the batch sentinel.  Column state (v, y, d, pred), row state (x),
// the free-row list, the search order cols[] and one row of the tile live in
// LDS (40 KiB).  Lane l handles columns / positions l, l + 64, ... of every
// K-wide pass; steps whose order matters (first index on ties, the swaps of
// the minimum-group gathering and of the row scans) are resolved per 64-wide
// chunk in increasing order with ballots, and each swap is replayed on cols[]
// by lane 0 in the reference's order.  Inputs outside the wave path's value
// range (|cost| > 1e15) run a lane-serial transcription instead.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "jv_batch.h"
#include "jv_common.h"
#include "jv_compact.h"
#include "wave.h"

namespace tmamd {
namespace {

constexpr int kCompactMaxK = 1024;
constexpr int kCompactChunks = kCompactMaxK / 64;
constexpr int kNoIndex = 0x7fffffff;

struct CompactLds {
    float v[kCompactMaxK];       // column duals
    float d[kCompactMaxK];       // path distances, by column
    float row[kCompactMaxK];     // one row of the padded tile
    int32_t y[kCompactMaxK];     // column -> row (colsol)
    int32_t x[kCompactMaxK];     // row -> column (rowsol)
    int32_t fr[kCompactMaxK];    // free rows
    int32_t pred[kCompactMaxK];  // path predecessors, by column
    int32_t cols[kCompactMaxK];  // search order: position -> column (collist)
    int32_t claims[kCompactMaxK];
    int32_t xmax[kCompactMaxK];
};

// The virtually padded K x K tile: 0 outside (N, M), non-finite -> sentinel.
struct TileView {
    const float *src;
    int N, M;
    float sentinel;
    __device__ __forceinline__ float at(int i, int j) const {
        if (i >= N || j >= M)
            return 0.f;
        const float c = src[(int64_t)i * M + j];
        return isfinite(c) ? c : sentinel;
    }
};

__device__ __forceinline__ void sync() { __syncthreads(); }

// Row i of the tile into L.row (all K columns).
__device__ __forceinline__ void stage_row(CompactLds &L, const TileView &C, int K, int i) {
    for (int j = lane_id(); j < K; j += 64)
        L.row[j] = C.at(i, j);
    sync();
}

// Exchange cols[a] and cols[b] (lane 0; the caller syncs before other lanes
// read cols[]).
__device__ __forceinline__ void swap_cols(CompactLds &L, int a, int b) {
    if (lane_id() == 0) {
        const int t = L.cols[a];
        L.cols[a] = L.cols[b];
        L.cols[b] = t;
    }
}

// Smallest index (0 .. 1023, kNoIndex when none) over the wave.
__device__ __forceinline__ int wave_min_index(int idx) { return uniform_i(wave_min_key(idx)); }

__device__ bool compact_large_solve(const int K, const int E, CompactLds &L, const TileView &C) {
    const int lane = lane_id();

    // ---- column reduction (:77-96): minimum of each column, first row on
    // ties (seeded by row 0); the largest column claiming a row keeps it
    float m[kCompactChunks];
    int im[kCompactChunks];
#pragma unroll
    for (int e = 0; e < kCompactChunks; ++e) {
        m[e] = 0.f;
        im[e] = 0;
        const int j = e * 64 + lane;
        if (e < E && j < K)
            m[e] = C.at(0, j);
    }
    // four rows per pass: all their loads are in flight before the folds
    int i = 1;
    for (; i + 4 <= K; i += 4) {
        float t[4][kCompactChunks];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int e = 0; e < kCompactChunks; ++e) {
                const int j = e * 64 + lane;
                t[r][e] = (e < E && j < K) ? C.at(i + r, j) : 0.f;
            }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int e = 0; e < kCompactChunks; ++e)
                if (t[r][e] < m[e]) {
                    m[e] = t[r][e];
                    im[e] = i + r;
                }
    }
    for (; i < K; ++i) {
#pragma unroll
        for (int e = 0; e < kCompactChunks; ++e) {
            const int j = e * 64 + lane;
            if (e < E && j < K) {
                const float val = C.at(i, j);
                if (val < m[e]) {
                    m[e] = val;
                    im[e] = i;
                }
            }
        }
    }
    for (int j = lane; j < K; j += 64) {
        L.xmax[j] = -1;
        L.claims[j] = 0;
    }
    sync();
#pragma unroll
    for (int e = 0; e < kCompactChunks; ++e) {
        const int j = e * 64 + lane;
        if (e < E && j < K) {
            atomicMax(&L.xmax[im[e]], j);
            atomicAdd(&L.claims[im[e]], 1);
        }
    }
    sync();
#pragma unroll
    for (int e = 0; e < kCompactChunks; ++e) {
        const int j = e * 64 + lane;
        if (e < E && j < K) {
            L.v[j] = m[e];
            L.y[j] = L.xmax[im[e]] == j ? im[e] : -1;
            L.x[j] = L.xmax[j];  // lane-chunk j doubles as row j here
        }
    }
    sync();

    // ---- free rows in row order, then the reduction transfer (:98-117):
    // each row claimed once lowers its column's dual by its smallest other
    // reduced cost (FLT_MAX when there is none), rows in increasing order
    int n_free = 0;
    const int max_key = fkey(kFltMax);
    for (int e = 0; e < E; ++e) {
        const int i = e * 64 + lane;
        const bool ok = i < K;
        const int cl = ok ? L.claims[i] : -1;
        const uint64_t freem = ballot(ok && cl == 0);
        const uint64_t once = ballot(ok && cl == 1);
        if (freem & (1ull << lane))
            L.fr[n_free + __builtin_popcountll(freem & ((1ull << lane) - 1))] = i;
        n_free += __builtin_popcountll(freem);
        uint64_t t = once;
        while (t) {
            const int row = e * 64 + first_lane(t);
            t &= t - 1;
            const int own = L.x[row];
            int kmin = kKeyNone;
            for (int j = lane; j < K; j += 64) {
                const float r = C.at(row, j) - L.v[j];
                if (j != own)
                    kmin = min(kmin, fkey(r));
            }
            kmin = uniform_i(wave_min_key(kmin));
            // the reduced costs are finite on this path, so the key's float
            // is the minimum (up to the sign of a zero, which no comparison sees)
            const float mn = kmin < max_key ? key_to_float(kmin) : kFltMax;
            sync();
            if (lane == 0)
                L.v[own] = L.v[own] - mn;
            sync();
        }
    }
    sync();

    // ---- augmenting row reduction (:119-166) ----
    const uint32_t guard = compact_arr_guard(K);
    uint32_t steps = 0;
    for (int round = 0; round < 2; ++round) {
        const int n_prev = n_free;
        int k = 0;
        n_free = 0;
        while (k < n_prev) {
            const int i = uniform_i(L.fr[k++]);
            if (++steps > guard)
                return false;
            // two smallest reduced costs of row i in (value, index) order
            int key[kCompactChunks];
            int lmin = kKeyNone;
#pragma unroll
            for (int e = 0; e < kCompactChunks; ++e) {
                const int j = e * 64 + lane;
                key[e] = kKeyNone;
                if (e < E && j < K) {
                    key[e] = fkey(C.at(i, j) - L.v[j]);
                    lmin = min(lmin, key[e]);
                }
            }
            const int k1 = uniform_i(wave_min_key(lmin));
            int first = kNoIndex, second = kNoIndex, rest = kKeyNone;
#pragma unroll
            for (int e = 0; e < kCompactChunks; ++e) {
                const int j = e * 64 + lane;
                if (key[e] == k1) {
                    if (first == kNoIndex)
                        first = j;
                    else if (second == kNoIndex)
                        second = j;
                }
            }
            const int j1 = wave_min_index(first);
            // second entry at the minimum, else the smallest key of the rest
            int cand = (first == j1) ? second : first;
            int j2 = wave_min_index(cand);
            int k2 = k1;
            if (j2 == kNoIndex) {
#pragma unroll
                for (int e = 0; e < kCompactChunks; ++e)
                    if (key[e] != k1)
                        rest = min(rest, key[e]);
                k2 = uniform_i(wave_min_key(rest));
                int at2 = kNoIndex;
#pragma unroll
                for (int e = 0; e < kCompactChunks; ++e) {
                    const int j = e * 64 + lane;
                    if (key[e] == k2 && k2 != kKeyNone && at2 == kNoIndex)
                        at2 = j;
                }
                j2 = wave_min_index(at2);
            }
            if (j2 == kNoIndex)
                return false;  // K >= 2 here, so this is unreachable
            const float u1 = key_to_float(k1);
            const float u2 = key_to_float(k2);
            int jsel = j1;
            int i0 = L.y[j1];
            const float vj1 = L.v[j1];
            const float lowered = vj1 - (u2 - u1);
            const bool lowers = lowered < vj1;
            if (!lowers && i0 >= 0) {
                jsel = j2;
                i0 = L.y[j2];
            }
            sync();
            if (lane == 0) {
                if (lowers)
                    L.v[j1] = lowered;
                L.x[i] = jsel;
                L.y[jsel] = i;
                if (i0 >= 0) {
                    if (lowers)
                        L.fr[k - 1] = i0;
                    else
                        L.fr[n_free] = i0;
                }
            }
            if (i0 >= 0) {
                if (lowers)
                    --k;
                else
                    ++n_free;
            }
            sync();
        }
    }

    // ---- augmentation (:168-251), one shortest-path search per free row ----
    for (int f = 0; f < n_free; ++f) {
        const int start = uniform_i(L.fr[f]);
        stage_row(L, C, K, start);
        for (int j = lane; j < K; j += 64) {
            L.d[j] = L.row[j] - L.v[j];
            L.pred[j] = start;
            L.cols[j] = j;
        }
        sync();
        int low = 0, up = 0, n_ready = 0, end = -1;
        float level = 0.f;
        while (end < 0) {
            if (low >= K)
                return false;  // no unassigned column reachable: cannot happen
            if (up == low) {
                // gather the columns at the new minimum into [low, up)
                // (:185-199): a smaller d restarts the group at low, an equal
                // one joins it; events in position order from a running
                // prefix minimum seeded by position low
                n_ready = low;
                int carry = fkey(L.d[L.cols[low]]);
                up = low + 1;
                for (int e = low / 64; e < E; ++e) {
                    const int p = e * 64 + lane;
                    const bool act = p > low && p < K;
                    const int kk = act ? fkey(L.d[L.cols[p]]) : kKeyNone;
                    const int before = min(carry, wave_shift_up_key(wave_prefix_min_key(kk)));
                    const uint64_t rec = ballot(act && kk < before);
                    const uint64_t tie = ballot(act && kk == before);
                    carry = min(carry, uniform_i(wave_min_key(kk)));
                    uint64_t ev = rec | tie;
                    while (ev) {
                        const int q = first_lane(ev);
                        ev &= ev - 1;
                        const int pos = e * 64 + q;
                        if ((rec >> q) & 1ull) {
                            swap_cols(L, pos, low);
                            up = low + 1;
                        } else {
                            if (pos != up)
                                swap_cols(L, pos, up);
                            ++up;
                        }
                    }
                    sync();
                }
                level = L.d[L.cols[low]];
                // the first unassigned column of the group ends the path (:200-206)
                for (int e = low / 64; e * 64 < up; ++e) {
                    const int p = e * 64 + lane;
                    const uint64_t open = ballot(p >= low && p < up && L.y[L.cols[p]] < 0);
                    if (open) {
                        end = L.cols[e * 64 + first_lane(open)];
                        break;
                    }
                }
            }
            if (end >= 0)
                break;
            // scan the row of the group's next column (:209-233)
            const int jq = L.cols[low];
            ++low;
            const int iq = L.y[jq];
            if (iq < 0)
                return false;  // group columns are assigned: cannot happen
            stage_row(L, C, K, iq);
            const float h = L.row[jq] - L.v[jq] - level;
            const int scan0 = up;
            for (int e = scan0 / 64; e < E && end < 0; ++e) {
                const int p = e * 64 + lane;
                const bool act = p >= scan0 && p < K;
                const int col = act ? L.cols[p] : 0;
                const float r = act ? (L.row[col] - L.v[col] - h) : 0.f;
                const bool better = act && r < L.d[col];
                const bool tie = better && r == level;
                const uint64_t ret = ballot(tie && L.y[col] < 0);
                const int lim = ret ? first_lane(ret) : 64;
                // the reference stops at the first such column: columns before
                // it are relaxed, it only gets its pred (:217-231)
                if (better && lane < lim) {
                    L.d[col] = r;
                    L.pred[col] = iq;
                }
                if (ret && lane == lim)
                    L.pred[col] = iq;
                uint64_t tm = ballot(tie && lane < lim);
                sync();
                while (tm) {
                    const int q = first_lane(tm);
                    tm &= tm - 1;
                    const int pos = e * 64 + q;
                    if (pos != up)
                        swap_cols(L, pos, up);
                    ++up;
                }
                if (ret)
                    end = readlane_i(col, lim);
                sync();
            }
        }
        // duals of the columns finished before the last group (:236-239)
        for (int p = lane; p < n_ready; p += 64) {
            const int j = L.cols[p];
            L.v[j] = L.v[j] + L.d[j] - level;
        }
        sync();
        // flip the assignment along the predecessors (:241-250)
        if (lane == 0) {
            int j = end, i = -1, hops = 0;
            do {
                if (j < 0 || j >= K || ++hops > K)
                    break;  // a broken chain: cannot happen
                i = L.pred[j];
                L.y[j] = i;
                const int prev = L.x[i];
                L.x[i] = j;
                j = prev;
            } while (i != start);
        }
        sync();
    }
    return true;
}

__global__ void __launch_bounds__(64)
jv_compact_large_kernel(const float *__restrict__ costs, int64_t B, int N, int M,
                        const JvStats *__restrict__ partial, int n_partial,
                        int64_t *__restrict__ out, uint32_t *__restrict__ status) {
    __shared__ CompactLds L;
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
    TileView C;
    C.src = costs + b * (int64_t)N * M;
    C.N = N;
    C.M = M;
    C.sentinel = any_finite ? (mx + 1.0f) * (float)(K + 1) : 1.0f;
    // wave path: every cost within +-1e15 (so every reduced cost stays far
    // below FLT_MAX); otherwise the lane-serial transcription
    const bool fast = !any_finite || (mx <= kFastRange && mn >= -kFastRange);
    bool ok;
    if (fast) {
        ok = compact_large_solve(K, E, L, C);
    } else {
        bool serial_ok = true;
        if (lane == 0) {
            auto cost = [&C](int i, int j) { return C.at(i, j); };
            serial_ok = compact_serial((uint32_t)K, cost, L.x, L.y, L.fr, L.pred, L.cols, L.v,
                                       L.d);
            L.claims[0] = serial_ok ? 1 : 0;
        }
        sync();
        ok = L.claims[0] != 0;
    }
    if (!ok) {
        if (lane == 0)
            atomicOr(&status[1], 1u);
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

int launch_jv_compact_large(const float *costs, int64_t B, int N, int M,
                            const JvStats *partial, int n_partial, int64_t *out,
                            uint32_t *status, hipStream_t stream) {
    hipLaunchKernelGGL(jv_compact_large_kernel, dim3((unsigned)B), dim3(64), 0, stream, costs,
                       B, N, M, partial, n_partial, out, status);
    return hipGetLastError() == hipSuccess ? kTmOk : kTmErrLaunch;
}

int jv_compact_max_k() { return kCompactMaxK; }

} // namespace tmamd
