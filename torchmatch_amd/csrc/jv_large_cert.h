// jv_large_cert.h -- certified shortest augmenting paths for 64 < K <= 1024
// and N <= M, four waves per problem (included by jv_large.hip).
//
// The exact replay of the reference's order (jv_large.hip) runs one wave per
// problem and spends most of its time in the augmenting row reduction, a
// sequential chain of row scans (C3: ~1,800 steps per problem).  When the
// optimum of the N x M problem is unique, every exact solver returns it, so
// this role takes a shorter road and then proves where it arrived:
//
// 1. Row minima: every row claims its smallest (sentinel-mapped) cost, the
//    highest claiming row keeps the column.  With v = 0 and u_i = that
//    minimum every reduced cost is >= 0 and the claims are tight.
// 2. One Dijkstra search per free row over the N x M problem (rectangular:
//    the padding rows of the reference's K x K tile are left out; a column
//    no real row takes is free).  Column j = e * 256 + w * 64 + l is held by
//    lane l of wave w in slot e (distance, order key, predecessor, dual, owner);
//    each step is a lane-local minimum over the slots, a wave minimum, and a
//    four-entry exchange through LDS (one barrier).  The scanned column's row
//    is read from memory and relaxes every open column:
//    r = ((c - v) - u) + level with u = c[i][j*] - v[j*].  Scanned columns'
//    duals move by d - level after each path (clamped at 0, so every dual of
//    a taken column stays <= the free columns' 0).
// 3. Certificate in float64.  With u_i = c[i][x_i] - v[x_i] and
//    r_ij = (c_ij - u_i) - v_j, the reference's padding rows (cost 0) get
//    dual 0 and reduced costs -v_j >= 0, zero on the free columns they hold.
//    Any assignment s of the K x K tile then costs cost(x) + sum of r over
//    its edges; the padding rows are interchangeable, so the free columns act
//    as one node F.  Let neg_i = max_j max(0, -r_ij) (float32 rounding of
//    the search leaves a few reduced costs ~1e-7 of the largest cost below
//    0).  If sum_i neg_i <= 2^-21 S and the graph with an edge x_i -> j
//    (j free: -> F) for each j != x_i with r_ij <= 2^-20 S and F -> j for
//    each taken column with -v_j <= 2^-20 S has no cycle, every other
//    assignment of the real rows costs more than cost(x) + 2^-21 S, S the
//    largest finite |cost| of the problem: x is the unique optimum by that
//    margin, and the reference's answer (jonker_dense_flat.h:27-274 on the
//    padded tile, ops.cpp:176-289) is x.
//
// C3 (64 x 512 x 768, 20 % +inf): every one of 640 problems (10 seeds) had
// the reference's mapping equal to the float64 optimum; 5 of them fail the
// certificate (near-ties below the margin) and keep the replay's answer.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "jv_common.h"
#include "wave.h"

namespace tmamd {
namespace cert {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxM = 1024;
constexpr int kMaxChunks64 = kMaxM / 64;  // row passes: lane l holds l, l + 64, ...
constexpr int kMaxEdges = 4096;
constexpr int kMaxPeelRounds = 512;

struct Lds {
    int32_t x[kMaxM];      // row -> column
    int32_t y[kMaxM];      // column -> row, -1 free
    int32_t pred[kMaxM];   // claims, then the searches' predecessors
    float v[kMaxM];        // duals for the certificate
    int32_t fr[kMaxM];     // free rows after the claims
    uint32_t edge[kMaxEdges];  // near-tight edges: src << 16 | dst, bit 31 = peeled
    int32_t indeg[kMaxM + 1];
    int32_t outdeg[kMaxM + 1];
    int4 slot[2][kWaves];  // per-wave minimum: key, column, owner, dual bits
    float wred[kWaves];
    int32_t n_edges;
    int32_t n_free;
};

__device__ __forceinline__ float fix(float raw, float sentinel) {
    return isfinite(raw) ? raw : sentinel;
}

__device__ __forceinline__ void add_edge(Lds &L, int src, int dst) {
    const int k = atomicAdd(&L.n_edges, 1);
    if (k < kMaxEdges)
        L.edge[k] = ((uint32_t)src << 16) | (uint32_t)dst;
}

// Rows split over the waves; lane l reads columns l, l + 64, ... (addresses
// clamped into the row, values past M ignored).
__device__ __forceinline__ void load_row64(const float *src, int M, int i,
                                           float (&raw)[kMaxChunks64]) {
    const float *row = src + (int64_t)i * M;
    const int lane = lane_id();
#pragma unroll
    for (int q = 0; q < kMaxChunks64; ++q)
        raw[q] = row[min(q * 64 + lane, M - 1)];
}

// Returns true when x (in L.x, rows < N) is certified.  C = ceil(M / 256).
template <int C>
__device__ __forceinline__ bool solve(Lds &L, const float *__restrict__ src, const int N,
                                      const int M, const float sentinel) {
    const int tid = threadIdx.x;
    const int lane = lane_id();
    const int w = tid >> 6;
    const int Q = (M + 63) >> 6;

    for (int k = tid; k < M; k += kThreads) {
        L.pred[k] = -1;
        L.x[k] = -1;
    }
    if (tid == 0)
        L.n_edges = 0;
    __syncthreads();

    // ---- 1. row minima and claims; largest finite |cost| ----
    float amax = 0.f;
    {
        float cur[kMaxChunks64];
        if (w < N)
            load_row64(src, M, w, cur);
        for (int i = w; i < N; i += kWaves) {
            float nxt[kMaxChunks64];
            load_row64(src, M, min(i + kWaves, N - 1), nxt);
            int kl = kKeyNone, ql = 0;
#pragma unroll
            for (int q = 0; q < kMaxChunks64; ++q) {
                if (q < Q && q * 64 + lane < M) {
                    const float raw = cur[q];
                    if (isfinite(raw))
                        amax = fmaxf(amax, fabsf(raw));
                    const int k = fkey(fix(raw, sentinel));
                    if (k < kl) {
                        kl = k;
                        ql = q;
                    }
                }
            }
            const int km = wave_min_key_s(kl);
            const int ln = first_lane(ballot(kl == km));
            const int jm = readlane_i(ql * 64 + lane, ln);
            if (lane == 0)
                atomicMax(&L.pred[jm], i);
#pragma unroll
            for (int q = 0; q < kMaxChunks64; ++q)
                cur[q] = nxt[q];
        }
    }
    amax = wave_max(amax);
    if (lane == 0)
        L.wred[w] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(L.wred[0], L.wred[1]), fmaxf(L.wred[2], L.wred[3]));
    for (int j = tid; j < M; j += kThreads) {
        const int i = L.pred[j];
        L.y[j] = i;
        if (i >= 0)
            L.x[i] = j;
    }
    __syncthreads();
    if (!(amax >= 1e-30f))
        return false;  // all zero: every assignment ties
    if (w == 0) {
        int n_free = 0;
        for (int base = 0; base < N; base += 64) {
            const int i = base + lane;
            const bool fre = i < N && L.x[i] < 0;
            const uint64_t m = ballot(fre);
            const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
            if (fre)
                L.fr[n_free + __builtin_popcountll(m & below)] = i;
            n_free += __builtin_popcountll(m);
        }
        if (lane == 0)
            L.n_free = n_free;
    }
    __syncthreads();
    const int n_free = L.n_free;

    // ---- 2. shortest augmenting paths ----
    float v[C], d[C];
    int key[C], pred[C], y[C];
#pragma unroll
    for (int e = 0; e < C; ++e) {
        const int j = e * kThreads + w * 64 + lane;
        v[e] = 0.f;
        y[e] = j < M ? L.y[j] : -1;
    }
    int par = 0;
    for (int t = 0; t < n_free; ++t) {
        const int f = L.fr[t];
        const float *rowf = src + (int64_t)f * M;
#pragma unroll
        for (int e = 0; e < C; ++e) {
            const int j = e * kThreads + w * 64 + lane;
            const float c = fix(rowf[min(j, M - 1)], sentinel);
            d[e] = c - v[e];
            key[e] = j < M ? fkey(d[e]) : kKeyNone;
            pred[e] = f;
        }
        uint32_t sc = 0;
        int sink = -1;
        float level = 0.f;
        for (int steps = 0; steps <= M; ++steps) {
            int kl = key[0], el = 0;
#pragma unroll
            for (int e = 1; e < C; ++e)
                if (key[e] < kl) {
                    kl = key[e];
                    el = e;
                }
            const int kw = wave_min_key_s(kl);
            const int ln = first_lane(ballot(kl == kw));
            int yl = y[0];
            float vl = v[0];
#pragma unroll
            for (int e = 1; e < C; ++e)
                if (el == e) {
                    yl = y[e];
                    vl = v[e];
                }
            if (lane == 0)
                L.slot[par][w] = make_int4(kw, readlane_i(el * kThreads + w * 64 + lane, ln),
                                           readlane_i(yl, ln), __float_as_int(readlane_f(vl, ln)));
            __syncthreads();
            int4 s = L.slot[par][0];
#pragma unroll
            for (int q = 1; q < kWaves; ++q) {
                const int4 o = L.slot[par][q];
                if (o.x < s.x || (o.x == s.x && o.y < s.y))
                    s = o;
            }
            par ^= 1;
            const int js = uniform_i(s.y), is = uniform_i(s.z);
            level = key_to_float(uniform_i(s.x));
            if (is < 0) {
                sink = js;
                break;
            }
#pragma unroll
            for (int e = 0; e < C; ++e)
                if (e * kThreads + w * 64 + lane == js) {
                    sc |= 1u << e;
                    key[e] = kKeyNone;
                }
            const float *row = src + (int64_t)is * M;
            const float u = fix(row[js], sentinel) - __int_as_float(uniform_i(s.w));
#pragma unroll
            for (int e = 0; e < C; ++e) {
                const int j = e * kThreads + w * 64 + lane;
                const float c = fix(row[min(j, M - 1)], sentinel);
                const float r = ((c - v[e]) - u) + level;
                if (key[e] != kKeyNone && r < d[e]) {
                    d[e] = r;
                    key[e] = fkey(r);
                    pred[e] = is;
                }
            }
        }
        if (sink < 0)
            return false;  // no free column reached (cannot happen for N <= M)
#pragma unroll
        for (int e = 0; e < C; ++e) {
            const int j = e * kThreads + w * 64 + lane;
            if ((sc >> e) & 1u)
                v[e] = fminf(v[e] + (d[e] - level), 0.f);
            if (((sc >> e) & 1u) || j == sink)
                L.pred[j] = pred[e];
        }
        __syncthreads();
        if (tid == 0) {
            int j = sink, i, hops = 0;
            do {
                i = L.pred[j];
                const int prev = L.x[i];
                L.y[j] = i;
                L.x[i] = j;
                j = prev;
            } while (i != f && j >= 0 && ++hops <= N);
        }
        __syncthreads();
#pragma unroll
        for (int e = 0; e < C; ++e) {
            const int j = e * kThreads + w * 64 + lane;
            y[e] = j < M ? L.y[j] : -1;
        }
    }

    // ---- 3. certificate ----
#pragma unroll
    for (int e = 0; e < C; ++e) {
        const int j = e * kThreads + w * 64 + lane;
        if (j < M)
            L.v[j] = v[e];
    }
    __syncthreads();
    const double tau = (double)amax * 0x1p-20;
    float negsum = 0.f;  // sum over this wave's rows of the row's largest -r
    {
        float cur[kMaxChunks64];
        if (w < N)
            load_row64(src, M, w, cur);
        for (int i = w; i < N; i += kWaves) {
            float nxt[kMaxChunks64];
            load_row64(src, M, min(i + kWaves, N - 1), nxt);
            const int xi = uniform_i(L.x[i]);
            const float cx = fix(src[(int64_t)i * M + xi], sentinel);
            const double u = (double)cx - (double)L.v[xi];
            float rn = 0.f;
#pragma unroll
            for (int q = 0; q < kMaxChunks64; ++q) {
                const int j = q * 64 + lane;
                if (q < Q && j < M) {
                    const double r = ((double)fix(cur[q], sentinel) - u) - (double)L.v[j];
                    rn = fmaxf(rn, (float)(-r));
                    if (j != xi && r <= tau)
                        add_edge(L, xi, L.y[j] >= 0 ? j : M);
                }
            }
            if (ballot(rn > 0.f))
                negsum += wave_max(rn);
#pragma unroll
            for (int q = 0; q < kMaxChunks64; ++q)
                cur[q] = nxt[q];
        }
    }
    for (int j = tid; j < M; j += kThreads)
        if (L.y[j] >= 0 && -(double)L.v[j] <= tau)
            add_edge(L, M, j);
    if (lane == 0)
        L.wred[w] = negsum;
    __syncthreads();
    // the float sums round: 1.0001 covers them many times over
    const float neg_total = (L.wred[0] + L.wred[1] + L.wred[2] + L.wred[3]) * 1.0001f;
    const int ne = L.n_edges;
    if (!(neg_total <= amax * 0x1p-21f) || ne > kMaxEdges)
        return false;
    // peel nodes without in- or out-edges until nothing is left (acyclic) or
    // nothing more goes (a cycle)
    for (int round = 0; round < kMaxPeelRounds; ++round) {
        for (int k = tid; k <= M; k += kThreads) {
            L.indeg[k] = 0;
            L.outdeg[k] = 0;
        }
        __syncthreads();
        for (int k = tid; k < ne; k += kThreads) {
            const uint32_t e = L.edge[k];
            if (!(e >> 31)) {
                atomicAdd(&L.outdeg[e >> 16], 1);
                atomicAdd(&L.indeg[e & 0xffffu], 1);
            }
        }
        __syncthreads();
        int removed = 0, alive = 0;
        for (int k = tid; k < ne; k += kThreads) {
            const uint32_t e = L.edge[k];
            if (!(e >> 31)) {
                if (L.indeg[e >> 16] == 0 || L.outdeg[e & 0xffffu] == 0) {
                    L.edge[k] = e | 0x80000000u;
                    removed = 1;
                } else {
                    alive = 1;
                }
            }
        }
        const int any_removed = __syncthreads_or(removed);
        const int any_alive = __syncthreads_or(alive);
        if (!any_alive)
            return true;
        if (!any_removed)
            return false;
    }
    return false;
}

} // namespace cert
} // namespace tmamd
