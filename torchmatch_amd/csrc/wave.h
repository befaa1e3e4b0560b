// wave.h -- wave64 building blocks for gfx950 (CDNA4).
//
// Everything here assumes a 64-lane wavefront with all lanes active, which is
// how every kernel in this library launches (block sizes are multiples of 64
// and no helper is called under divergent control flow).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tmamd {

// DPP control words (GFX9 encoding, valid on gfx950).
enum : int {
    kDppQuadXor1 = 0xB1,       // quad_perm:[1,0,3,2]
    kDppQuadXor2 = 0x4E,       // quad_perm:[2,3,0,1]
    kDppRowShr1 = 0x111,
    kDppRowShr2 = 0x112,
    kDppRowShr4 = 0x114,
    kDppRowShr8 = 0x118,
    kDppWaveShr1 = 0x138,
    kDppRowMirror = 0x140,
    kDppRowHalfMirror = 0x141,
    kDppRowBcast15 = 0x142,
    kDppRowBcast31 = 0x143,
};

__device__ __forceinline__ int lane_id() { return (int)__lane_id(); }

__device__ __forceinline__ uint64_t ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }

__device__ __forceinline__ int readlane_i(int x, int lane) {
    return __builtin_amdgcn_readlane(x, lane);
}
__device__ __forceinline__ float readlane_f(float x, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}
__device__ __forceinline__ int uniform_i(int x) { return __builtin_amdgcn_readfirstlane(x); }

// v_writelane_b32: `old` with lane `lane` (uniform) replaced by `val` (uniform).
// This clang has no builtin; the intrinsic is declared by its LLVM name.
extern "C" __device__ int tmamd_llvm_writelane_i32(int val, int lane, int old) __asm(
    "llvm.amdgcn.writelane.i32");
__device__ __forceinline__ uint32_t writelane_i(int val, int lane, uint32_t old) {
    return (uint32_t)tmamd_llvm_writelane_i32(val, lane, (int)old);
}
__device__ __forceinline__ float uniform_f(float x) {
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
}

// Move `src` through a DPP pattern; lanes whose source is outside the pattern
// keep `identity`.
template <int CTRL, int ROW_MASK = 0xF, int BANK_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float identity, float src) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(identity),
                                                      __float_as_int(src), CTRL,
                                                      ROW_MASK, BANK_MASK, false));
}

// Minimum over the whole wave, returned uniformly (every lane gets it).  Exact:
// min is order independent.  NaN lanes must not occur (callers guarantee).
__device__ __forceinline__ float wave_min(float x) {
    const float inf = __int_as_float(0x7f800000);
    x = fminf(x, dpp_f<kDppQuadXor1>(inf, x));
    x = fminf(x, dpp_f<kDppQuadXor2>(inf, x));
    x = fminf(x, dpp_f<kDppRowHalfMirror>(inf, x));
    x = fminf(x, dpp_f<kDppRowMirror>(inf, x));
    const float a = fminf(readlane_f(x, 0), readlane_f(x, 16));
    const float b = fminf(readlane_f(x, 32), readlane_f(x, 48));
    return fminf(a, b);
}

// Maximum over the whole wave (uniform result).
__device__ __forceinline__ float wave_max(float x) {
    const float ninf = __int_as_float(0xff800000);
    x = fmaxf(x, dpp_f<kDppQuadXor1>(ninf, x));
    x = fmaxf(x, dpp_f<kDppQuadXor2>(ninf, x));
    x = fmaxf(x, dpp_f<kDppRowHalfMirror>(ninf, x));
    x = fmaxf(x, dpp_f<kDppRowMirror>(ninf, x));
    const float a = fmaxf(readlane_f(x, 0), readlane_f(x, 16));
    const float b = fmaxf(readlane_f(x, 32), readlane_f(x, 48));
    return fmaxf(a, b);
}

// Smallest and second smallest value of the wave as a multiset (if the
// minimum occurs twice, both results are equal).  Uniform results.
__device__ __forceinline__ void wave_min2(float x, float &m1, float &m2) {
    const float inf = __int_as_float(0x7f800000);
    float a = x, b = inf;
#define TMAMD_MIN2_STEP(CTRL)                                   \
    {                                                           \
        const float pa = dpp_f<CTRL>(inf, a);                   \
        const float pb = dpp_f<CTRL>(inf, b);                   \
        const float lo = fminf(a, pa);                          \
        b = fminf(fmaxf(a, pa), fminf(b, pb));                  \
        a = lo;                                                 \
    }
    TMAMD_MIN2_STEP(kDppQuadXor1)
    TMAMD_MIN2_STEP(kDppQuadXor2)
    TMAMD_MIN2_STEP(kDppRowHalfMirror)
    TMAMD_MIN2_STEP(kDppRowMirror)
#undef TMAMD_MIN2_STEP
    // merge the four 16-lane rows
    float r1 = readlane_f(a, 0), r2 = readlane_f(b, 0);
#pragma unroll
    for (int row = 16; row < 64; row += 16) {
        const float q1 = readlane_f(a, row), q2 = readlane_f(b, row);
        const float lo = fminf(r1, q1);
        r2 = fminf(fmaxf(r1, q1), fminf(r2, q2));
        r1 = lo;
    }
    m1 = r1;
    m2 = r2;
}

// Inclusive prefix minimum across lanes 0..63 (lane p gets min of lanes 0..p).
__device__ __forceinline__ float wave_prefix_min(float x) {
    const float inf = __int_as_float(0x7f800000);
    x = fminf(x, dpp_f<kDppRowShr1>(inf, x));
    x = fminf(x, dpp_f<kDppRowShr2>(inf, x));
    x = fminf(x, dpp_f<kDppRowShr4>(inf, x));
    x = fminf(x, dpp_f<kDppRowShr8>(inf, x));
    x = fminf(x, dpp_f<kDppRowBcast15, 0xA>(inf, x));
    x = fminf(x, dpp_f<kDppRowBcast31, 0xC>(inf, x));
    return x;
}

// Value of lane p-1 (lane 0 gets `identity`).
__device__ __forceinline__ float wave_shift_up(float identity, float x) {
    return dpp_f<kDppWaveShr1>(identity, x);
}

__device__ __forceinline__ int first_lane(uint64_t m) { return (int)__builtin_ctzll(m); }
// Number of lanes below this one whose bit is set in m.
__device__ __forceinline__ int lanes_below(uint64_t m) {
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                          __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}
__device__ __forceinline__ int last_lane(uint64_t m) { return 63 - (int)__builtin_clzll(m); }

} // namespace tmamd

namespace tmamd {

// ---- integer-key reductions (no NaN canonicalisation, full-rate VALU) ------

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// Order-preserving int32 key of a float that is not NaN: key(a) < key(b) iff
// a < b, and -0.0 / +0.0 share one key (a + 0.0f turns -0.0 into +0.0), so
// key equality is float equality.
__device__ __forceinline__ int fkey(float f) {
    const int b = __float_as_int(f + 0.0f);
    return b ^ ((b >> 31) & 0x7fffffff);
}
constexpr int kKeyNone = 0x7fffffff;  // a NaN bit pattern: above every key

// fkey without the -0.0 fold: order-preserving for every non-NaN float, with
// -0.0 just below +0.0 (for minima whose ties need not be exact)
__device__ __forceinline__ int fkey_signed(float f) {
    const int b = __float_as_int(f);
    return b ^ ((b >> 31) & 0x7fffffff);
}

// DPP move for patterns in which every lane has a source lane (quad_perm,
// row mirrors), so the old value never shows and the move can fold into the
// consuming ALU op.
template <int CTRL>
__device__ __forceinline__ int dpp_full(int x) {
    return __builtin_amdgcn_mov_dpp(x, CTRL, 0xF, 0xF, true);
}

// Merge two (smallest, second smallest) multiset pairs.
__device__ __forceinline__ void pair_merge(int &a, int &b, int pa, int pb) {
    const int lo = min(a, pa);
    b = min(max(a, pa), min(b, pb));
    a = lo;
}

// Smallest and second smallest key of the wave (as a multiset), returned in
// every lane.  Butterfly: 4 DPP stages inside each 16-lane row, then the
// gfx950 row-swap permutes for the 16- and 32-lane exchanges.
__device__ __forceinline__ void wave_min2_key(int key, int &k1, int &k2) {
    int a = key, b = kKeyNone;
    pair_merge(a, b, dpp_full<kDppQuadXor1>(a), dpp_full<kDppQuadXor1>(b));
    pair_merge(a, b, dpp_full<kDppQuadXor2>(a), dpp_full<kDppQuadXor2>(b));
    pair_merge(a, b, dpp_full<kDppRowHalfMirror>(a), dpp_full<kDppRowHalfMirror>(b));
    pair_merge(a, b, dpp_full<kDppRowMirror>(a), dpp_full<kDppRowMirror>(b));
    u32x2 sa = __builtin_amdgcn_permlane16_swap((unsigned)a, (unsigned)a, false, false);
    u32x2 sb = __builtin_amdgcn_permlane16_swap((unsigned)b, (unsigned)b, false, false);
    a = (int)sa[0];
    b = (int)sb[0];
    pair_merge(a, b, (int)sa[1], (int)sb[1]);
    sa = __builtin_amdgcn_permlane32_swap((unsigned)a, (unsigned)a, false, false);
    sb = __builtin_amdgcn_permlane32_swap((unsigned)b, (unsigned)b, false, false);
    a = (int)sa[0];
    b = (int)sb[0];
    pair_merge(a, b, (int)sa[1], (int)sb[1]);
    k1 = a;
    k2 = b;
}

// Smallest key of the wave, returned in every lane.
__device__ __forceinline__ int wave_min_key(int key) {
    int a = key;
    a = min(a, dpp_full<kDppQuadXor1>(a));
    a = min(a, dpp_full<kDppQuadXor2>(a));
    a = min(a, dpp_full<kDppRowHalfMirror>(a));
    a = min(a, dpp_full<kDppRowMirror>(a));
    u32x2 s = __builtin_amdgcn_permlane16_swap((unsigned)a, (unsigned)a, false, false);
    a = min((int)s[0], (int)s[1]);
    s = __builtin_amdgcn_permlane32_swap((unsigned)a, (unsigned)a, false, false);
    return min((int)s[0], (int)s[1]);
}

// Smallest key of the wave as a scalar: the 16-lane rows reduce with DPP
// butterflies, row_bcast:15 / row_bcast:31 carry the minima up to lane 63,
// which is read out (152 cycles per dependent call against 176 for
// wave_min_key + readfirstlane, measured on gfx950).
__device__ __forceinline__ int wave_min_key_s(int key) {
    int a = key;
    a = min(a, dpp_full<kDppQuadXor1>(a));
    a = min(a, dpp_full<kDppQuadXor2>(a));
    a = min(a, dpp_full<kDppRowHalfMirror>(a));
    a = min(a, dpp_full<kDppRowMirror>(a));
    a = min(a, __builtin_amdgcn_update_dpp(kKeyNone, a, kDppRowBcast15, 0xA, 0xF, false));
    a = min(a, __builtin_amdgcn_update_dpp(kKeyNone, a, kDppRowBcast31, 0xC, 0xF, false));
    return __builtin_amdgcn_readlane(a, 63);
}

// Inclusive prefix minimum of keys across lanes 0..63.
__device__ __forceinline__ int wave_prefix_min_key(int x) {
    const int none = kKeyNone;
    x = min(x, __builtin_amdgcn_update_dpp(none, x, kDppRowShr1, 0xF, 0xF, false));
    x = min(x, __builtin_amdgcn_update_dpp(none, x, kDppRowShr2, 0xF, 0xF, false));
    x = min(x, __builtin_amdgcn_update_dpp(none, x, kDppRowShr4, 0xF, 0xF, false));
    x = min(x, __builtin_amdgcn_update_dpp(none, x, kDppRowShr8, 0xF, 0xF, false));
    x = min(x, __builtin_amdgcn_update_dpp(none, x, kDppRowBcast15, 0xA, 0xF, false));
    x = min(x, __builtin_amdgcn_update_dpp(none, x, kDppRowBcast31, 0xC, 0xF, false));
    return x;
}

// Key of lane p-1 (lane 0 gets kKeyNone).
__device__ __forceinline__ int wave_shift_up_key(int x) {
    return __builtin_amdgcn_update_dpp(kKeyNone, x, kDppWaveShr1, 0xF, 0xF, false);
}

// Register-resident 64-entry column (lane j keeps c[0..63][j]); reads take a
// wave-uniform row index and compile to indexed VGPR moves.
typedef float f32x32 __attribute__((ext_vector_type(32)));
struct Col64 {
    f32x32 lo, hi;
    __device__ __forceinline__ float get(int i) const {  // i uniform, 0 <= i < 64
        const int k = i & 31;
        const float a = lo[k], b = hi[k];
        return (i < 32) ? a : b;
    }
    __device__ __forceinline__ void set(int i, float x) {  // i a constant, 0 <= i < 64
        if (i < 32)
            lo[i] = x;
        else
            hi[i - 32] = x;
    }
};

// Lane `lane` (uniform) of a float64.
__device__ __forceinline__ double readlane_d(double x, int lane) {
    const long long b = __double_as_longlong(x);
    const int lo = __builtin_amdgcn_readlane((int)(b & 0xffffffffll), lane);
    const int hi = __builtin_amdgcn_readlane((int)(b >> 32), lane);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

} // namespace tmamd

namespace tmamd {
// Inverse of fkey (the transform is an involution on bit patterns); exact for
// every float except -0.0, which fkey folds into +0.0.
__device__ __forceinline__ float key_to_float(int k) {
    return __int_as_float(k ^ ((k >> 31) & 0x7fffffff));
}
} // namespace tmamd

namespace tmamd {
// Float butterfly reductions over the whole wave, result in every lane:
// 4 DPP stages inside each 16-lane row, then the gfx950 row swaps.  No LDS
// (unlike __shfl_xor, which goes through ds_bpermute).
template <int CTRL>
__device__ __forceinline__ float dpp_full_f(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

__device__ __forceinline__ float row_swap16_pair(float x, float &other) {
    const u32x2 s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                     false, false);
    other = __uint_as_float(s[1]);
    return __uint_as_float(s[0]);
}

__device__ __forceinline__ float row_swap32_pair(float x, float &other) {
    const u32x2 s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                     false, false);
    other = __uint_as_float(s[1]);
    return __uint_as_float(s[0]);
}

__device__ __forceinline__ float wave_sum_all(float x) {
    x += dpp_full_f<kDppQuadXor1>(x);
    x += dpp_full_f<kDppQuadXor2>(x);
    x += dpp_full_f<kDppRowHalfMirror>(x);
    x += dpp_full_f<kDppRowMirror>(x);
    float o;
    float a = row_swap16_pair(x, o);
    x = a + o;
    a = row_swap32_pair(x, o);
    return a + o;
}

// float64 DPP move: the two 32-bit halves moved with the same control.
template <int CTRL>
__device__ __forceinline__ double dpp_full_d(double x) {
    const uint64_t u = (uint64_t)__double_as_longlong(x);
    const int lo = __builtin_amdgcn_mov_dpp((int)(uint32_t)u, CTRL, 0xF, 0xF, true);
    const int hi = __builtin_amdgcn_mov_dpp((int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, true);
    return __longlong_as_double((long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
}

// Sum over the whole wave in float64 (uniform result), the same butterfly as
// wave_sum_all.  Adding 64 float32 lane sums in float32 loses the lanes that
// fall below half an ulp of their partner, always downward: a sum whose
// lanes span many orders of magnitude comes out biased low.
__device__ __forceinline__ double wave_sum_all_d(double x) {
    x += dpp_full_d<kDppQuadXor1>(x);
    x += dpp_full_d<kDppQuadXor2>(x);
    x += dpp_full_d<kDppRowHalfMirror>(x);
    x += dpp_full_d<kDppRowMirror>(x);
    const uint64_t u = (uint64_t)__double_as_longlong(x);
    u32x2 lo = __builtin_amdgcn_permlane16_swap((uint32_t)u, (uint32_t)u, false, false);
    u32x2 hi = __builtin_amdgcn_permlane16_swap((uint32_t)(u >> 32), (uint32_t)(u >> 32), false,
                                                false);
    x = __longlong_as_double((long long)(((uint64_t)hi[0] << 32) | lo[0])) +
        __longlong_as_double((long long)(((uint64_t)hi[1] << 32) | lo[1]));
    const uint64_t v = (uint64_t)__double_as_longlong(x);
    lo = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
    hi = __builtin_amdgcn_permlane32_swap((uint32_t)(v >> 32), (uint32_t)(v >> 32), false, false);
    return __longlong_as_double((long long)(((uint64_t)hi[0] << 32) | lo[0])) +
           __longlong_as_double((long long)(((uint64_t)hi[1] << 32) | lo[1]));
}

__device__ __forceinline__ float wave_max_all(float x) {
    x = fmaxf(x, dpp_full_f<kDppQuadXor1>(x));
    x = fmaxf(x, dpp_full_f<kDppQuadXor2>(x));
    x = fmaxf(x, dpp_full_f<kDppRowHalfMirror>(x));
    x = fmaxf(x, dpp_full_f<kDppRowMirror>(x));
    float o;
    float a = row_swap16_pair(x, o);
    x = fmaxf(a, o);
    a = row_swap32_pair(x, o);
    return fmaxf(a, o);
}
} // namespace tmamd
