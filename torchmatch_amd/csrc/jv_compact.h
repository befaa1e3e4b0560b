// jv_compact.h -- pieces of the compact JV solver shared by the K <= 64
// (jv_batch.hip) and 64 < K <= 1024 (jv_large.hip) kernels.
//
// jonker_compact_core.h:20-252 (torchmatch's square JV behind the CPU op
// assignment::jonker_compact_batch) has its own tie and ordering rules:
//   * column reduction from the last column, minima seeded by row 0, the
//     first column (in that order) to reach a row keeps it;
//   * reduction transfer with FLT_MAX as the starting minimum;
//   * augmenting row reduction without an iteration cap, the second minimum
//     seeded by FLT_MAX, the displaced owner pushed back at the read position
//     (lowered dual) or appended to the next round;
//   * augmentation: the FIRST unassigned column of a new minimum group ends
//     the path, and the finished columns' duals become (v + d) - min.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace tmamd {

constexpr float kFltMax = 3.402823466e38f;  // numeric_limits<float>::max()

// Iteration guard of the augmenting row reduction, which has no cap in the
// reference: measured runs stay below 0.7 K^2 steps (uniform, tied, masked
// and Gaussian costs, K = 64 .. 1024), so tripping it means a runaway, which
// is reported instead of spinning.
__device__ __forceinline__ uint32_t compact_arr_guard(int K) {
    return 8u * (uint32_t)K * (uint32_t)K + 65536u;
}

// The compact solver runs on the dense wave solvers (with its switches) when
// every cost of the padded tile, the +inf sentinel included, lies within
// +-1e12: the duals then stay far below LARGE (1e18), where the dense code's
// LARGE-specific branches would part from the compact rules (FLT_MAX seeds).
// Other inputs take compact_serial below.
constexpr float kCompactWaveRange = 1e12f;

__device__ __forceinline__ bool compact_wave_range(bool any_finite, float mx, float mn,
                                                   bool has_inf, float sentinel) {
    if (any_finite && (mx > kCompactWaveRange || mn < -kCompactWaveRange))
        return false;
    return !has_inf || fabsf(sentinel) <= kCompactWaveRange;
}

// Lane-serial transcription of jonker_compact_kernel<int32_t, float>
// (jonker_compact_core.h:20-252) on the padded n x n tile c(i, j), with the
// reference's scratch arrays (each of length >= n).  Exact for any finite
// input; used where the wave paths' value range does not hold.  Returns
// false when the iteration guard trips or the reference would index
// colsol[-1] (no second minimum below FLT_MAX).
template <typename Cost>
__device__ bool compact_serial(uint32_t n, Cost c, int32_t *x, int32_t *y, int32_t *fr,
                               int32_t *pred, int32_t *cols, float *v, float *d) {
    for (uint32_t i = 0; i < n; ++i)
        fr[i] = 0;
    // column reduction (:77-96)
    for (int32_t j = (int32_t)n - 1; j >= 0; --j) {
        float m = c(0, j);
        int32_t im = 0;
        for (uint32_t i = 1; i < n; ++i) {
            const float val = c((int)i, j);
            if (val < m) {
                m = val;
                im = (int32_t)i;
            }
        }
        v[j] = m;
        if (++fr[im] == 1) {
            x[im] = j;
            y[j] = im;
        } else {
            y[j] = -1;
        }
    }
    // reduction transfer (:98-117); fr[] holds the claim counts until read
    uint32_t n_free = 0;
    for (uint32_t i = 0; i < n; ++i) {
        const int32_t claims = fr[i];
        if (claims == 0) {
            fr[n_free++] = (int32_t)i;
        } else if (claims == 1) {
            const int32_t jx = x[i];
            float m = kFltMax;
            for (uint32_t j = 0; j < n; ++j) {
                const float r = c((int)i, (int)j) - v[j];
                if ((int32_t)j != jx && r < m)
                    m = r;
            }
            v[jx] = v[jx] - m;
        }
    }
    // augmenting row reduction (:119-166)
    const uint32_t guard = compact_arr_guard((int)n);
    uint32_t steps = 0;
    for (int round = 0; round < 2; ++round) {
        const uint32_t n_prev = n_free;
        uint32_t k = 0;
        n_free = 0;
        while (k < n_prev) {
            const int32_t i = fr[k++];
            if (++steps > guard)
                return false;
            float u1 = c(i, 0) - v[0], u2 = kFltMax;
            int32_t j1 = 0, j2 = -1;
            for (uint32_t j = 1; j < n; ++j) {
                const float h = c(i, (int)j) - v[j];
                if (!(h < u2))
                    continue;
                if (h >= u1) {
                    u2 = h;
                    j2 = (int32_t)j;
                } else {
                    u2 = u1;
                    j2 = j1;
                    u1 = h;
                    j1 = (int32_t)j;
                }
            }
            int32_t i0 = y[j1];
            const float lowered = v[j1] - (u2 - u1);
            const bool lowers = lowered < v[j1];
            if (lowers) {
                v[j1] = lowered;
            } else if (i0 >= 0) {
                if (j2 < 0)
                    return false;  // the reference would read colsol[-1]
                j1 = j2;
                i0 = y[j2];
            }
            x[i] = j1;
            y[j1] = i;
            if (i0 >= 0) {
                if (lowers)
                    fr[--k] = i0;
                else
                    fr[n_free++] = i0;
            }
        }
    }
    // augmentation (:168-251)
    for (uint32_t f = 0; f < n_free; ++f) {
        const int32_t start = fr[f];
        for (uint32_t j = 0; j < n; ++j) {
            d[j] = c(start, (int)j) - v[j];
            pred[j] = start;
            cols[j] = (int32_t)j;
        }
        uint32_t low = 0, up = 0;
        int32_t last = 0, end = -1;
        float level = 0.f;
        while (end < 0) {
            if (low >= n)
                return false;
            if (up == low) {
                last = (int32_t)low - 1;
                level = d[cols[up++]];
                for (uint32_t k = up; k < n; ++k) {
                    const int32_t j = cols[k];
                    const float h = d[j];
                    if (h <= level) {
                        if (h < level) {
                            up = low;
                            level = h;
                        }
                        cols[k] = cols[up];
                        cols[up++] = j;
                    }
                }
                for (uint32_t k = low; k < up; ++k)
                    if (y[cols[k]] < 0) {
                        end = cols[k];
                        break;
                    }
            }
            if (end >= 0)
                break;
            const int32_t jq = cols[low++];
            const int32_t iq = y[jq];
            const float h = c(iq, jq) - v[jq] - level;
            for (uint32_t k = up; k < n; ++k) {
                const int32_t j = cols[k];
                const float r = c(iq, j) - v[j] - h;
                if (!(r < d[j]))
                    continue;
                pred[j] = iq;
                if (r == level) {
                    if (y[j] < 0) {
                        end = j;
                        break;
                    }
                    cols[k] = cols[up];
                    cols[up++] = j;
                }
                d[j] = r;
            }
        }
        for (int32_t k = 0; k <= last; ++k) {
            const int32_t j = cols[k];
            v[j] = v[j] + d[j] - level;
        }
        int32_t i;
        uint32_t hops = 0;
        do {
            i = pred[end];
            y[end] = i;
            const int32_t j = end;
            end = x[i];
            x[i] = j;
            if (++hops > n)
                return false;
        } while (i != start);
    }
    return true;
}

} // namespace tmamd
