// ref_harness.cpp -- C entry points around the reference's own compiled
// jonker_dense_core.cpp and header-only jonker_compact_core.h, for building
// oracle/_ref/libjv_ref.so.
//
// TEST INFRASTRUCTURE ONLY (parity checker / CPU baseline, never shipped).
// The solve itself is the reference's code, compiled from
// /root/reference/sources/torchmatch/assignment/cpu/jonker_dense_core.cpp by
// oracle/Makefile.  This file only supplies the batch driver that ops.cpp
// wraps around it (ops.cpp:176-289: serial sentinel pass, per-problem K x K
// padding with +inf -> sentinel and zero padding, parallel loop over the
// batch, padded columns -> -1).  It has no torch dependency so it loads with
// ctypes on a box that does not have the reference checked out.
#include "jonker_compact_core.h"
#include "jonker_dense_core.h"

#include <cmath>
#include <cstdint>
#include <limits>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

int sentinel_of(const float *data, int64_t count, int K, float *out) {
    float mx = std::numeric_limits<float>::lowest();
    bool any = false, nan_seen = false, neg_inf_seen = false;
    for (int64_t k = 0; k < count; ++k) {
        const float x = data[k];
        if (std::isnan(x))
            nan_seen = true;
        else if (x == -std::numeric_limits<float>::infinity())
            neg_inf_seen = true;
        else if (std::isfinite(x)) {
            mx = x > mx ? x : mx;
            any = true;
        }
    }
    if (nan_seen)
        return 1;
    if (neg_inf_seen)
        return 2;
    *out = any ? (mx + 1.0f) * static_cast<float>(K + 1) : 1.0f;
    return 0;
}

using SquareSolver = int (*)(const float *, int, int64_t *, int64_t *);

int batch_driver(const float *costs, int64_t B, int32_t N, int32_t M, int64_t *out,
                 int threads, SquareSolver solve) {
    if (B == 0 || N == 0 || M == 0) {
        for (int64_t k = 0; k < B * static_cast<int64_t>(N); ++k)
            out[k] = -1;
        return 0;
    }
    const int K = N > M ? N : M;
    float sentinel = 1.0f;
    const int rc = sentinel_of(costs, B * static_cast<int64_t>(N) * M, K, &sentinel);
    if (rc != 0)
        return rc;
#ifdef _OPENMP
    if (threads <= 0)
        threads = omp_get_max_threads();
#pragma omp parallel num_threads(threads)
#endif
    {
        std::vector<float> tile(static_cast<size_t>(K) * K);
        std::vector<int64_t> rtc(K), ctr(K);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int64_t b = 0; b < B; ++b) {
            const float *src = costs + b * static_cast<int64_t>(N) * M;
            for (int i = 0; i < K; ++i)
                for (int j = 0; j < K; ++j) {
                    float val = 0.0f;
                    if (i < N && j < M) {
                        val = src[static_cast<size_t>(i) * M + j];
                        if (!std::isfinite(val))
                            val = sentinel;
                    }
                    tile[static_cast<size_t>(i) * K + j] = val;
                }
            const int src_rc = solve(tile.data(), K, rtc.data(), ctr.data());
            int64_t *ob = out + b * N;
            for (int i = 0; i < N; ++i) {
                const int64_t j = src_rc == 0 ? rtc[i] : -1;
                ob[i] = (j >= 0 && j < M) ? j : -1;
            }
        }
    }
    (void)threads;
    return 0;
}

} // namespace

extern "C" int ref_jv_dense_batch_f32(const float *costs, int64_t B, int32_t N,
                                      int32_t M, int64_t *out, int threads) {
    return batch_driver(costs, B, N, M, out, threads,
                        &match_jonker::detail::jonker_dense_solve_square_f32);
}

// jonker_compact_batch (ops.cpp:431-433): the same driver around the
// compact square solver (jonker_compact_core.h:279-301).
extern "C" int ref_jv_compact_batch_f32(const float *costs, int64_t B, int32_t N,
                                        int32_t M, int64_t *out, int threads) {
    return batch_driver(costs, B, N, M, out, threads,
                        &match_jonker::detail::jonker_compact_solve_square_f32);
}
