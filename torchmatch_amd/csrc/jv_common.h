// jv_common.h -- device helpers shared by the JV kernels (jv_batch.hip,
// jv_large.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "jv_batch.h"
#include "wave.h"

namespace tmamd {

constexpr float kLarge = 1e18f;      // jonker_dense_flat.h:22-23 (LARGE_V<float>)
constexpr float kFastRange = 1e15f;  // wave paths valid for |cost| <= this

__device__ __forceinline__ float finf() { return __int_as_float(0x7f800000); }

// Raise the internal-error word of the status pair.  Every writer stores the
// same value, so a plain store suffices; it also works when the status words
// live in host-mapped pinned memory, where device atomics are not assumed.
__device__ __forceinline__ void raise_guard(uint32_t *status) {
    __hip_atomic_store(&status[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Fold the per-block partials (uniform result in every lane of the wave).
__device__ __forceinline__ void fold_stats(const JvStats *__restrict__ partial, int n_partial,
                                           float &mx, float &mn, uint32_t &flags) {
    mx = -finf();
    mn = finf();
    uint32_t f = 0;
    for (int k = lane_id(); k < n_partial; k += 64) {
        mx = fmaxf(mx, partial[k].max_finite);
        mn = fminf(mn, partial[k].min_finite);
        f |= partial[k].flags;
    }
    mx = wave_max(mx);
    mn = wave_min(mn);
    flags = 0;
#pragma unroll
    for (int bit = 0; bit < 5; ++bit)
        if (ballot((f >> bit) & 1u))
            flags |= 1u << bit;
}


} // namespace tmamd
