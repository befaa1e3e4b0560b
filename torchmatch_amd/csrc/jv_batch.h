// jv_batch.h -- internal declarations shared by the JV kernels and the C ABI.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include "../../include/torchmatch_amd.h"

namespace tmamd {

constexpr int kTmOk = TM_OK;
constexpr int kTmErrInvalidArgument = TM_ERR_INVALID_ARGUMENT;
constexpr int kTmErrUnsupportedShape = TM_ERR_UNSUPPORTED_SHAPE;
constexpr int kTmErrWorkspace = TM_ERR_WORKSPACE;
constexpr int kTmErrLaunch = TM_ERR_LAUNCH;

constexpr uint32_t kJvFlagNan = TM_JV_FLAG_NAN;
constexpr uint32_t kJvFlagNegInf = TM_JV_FLAG_NEG_INF;
constexpr uint32_t kJvFlagPosInf = TM_JV_FLAG_POS_INF;
constexpr uint32_t kJvFlagAnyFinite = TM_JV_FLAG_ANY_FINITE;
constexpr uint32_t kJvFlagNegZero = TM_JV_FLAG_NEG_ZERO;
constexpr uint32_t kJvFlagDone = TM_JV_FLAG_DONE;

// Upper bound on the blocks of the statistics pass (and so on the partial
// records every solve workgroup folds).
constexpr int kJvMaxStatBlocks = 256;

struct JvStats {
    float max_finite;
    float min_finite;
    uint32_t flags;
    uint32_t info;  // unused (0)
};

// The fused path also keeps one summary byte per problem: bits 0-4 the
// TM_JV_FLAG_* of its tile, then the bits below.
constexpr uint32_t kJvRecDeferred = 1u << 5;  // holds +inf: solved once the batch is folded
constexpr uint32_t kJvRecReplayed = 1u << 6;  // left the certified path for the exact replay
constexpr uint32_t kJvRecGuard = 1u << 7;     // a solve hit its iteration guard

// K in (64, jv_large_max_k()]: one workgroup per problem, cost read from
// global memory (jv_large.hip).  prep_ws: nullptr, or jv_large_prep_bytes of
// device memory for the prefill (column minima and row caches built by
// many-wave launches before the solve; the same result either way).
int launch_jv_large(const float *costs, int64_t B, int N, int M, const JvStats *partial,
                    int n_partial, void *prep_ws, int64_t *out, uint32_t *status,
                    hipStream_t stream);
int jv_large_max_k();
size_t jv_large_prep_bytes(int64_t B, int N, int M);

// Compact solver (assignment::jonker_compact_batch) for K in (64,
// jv_compact_max_k()] (jv_large.hip).
int launch_jv_compact_large(const float *costs, int64_t B, int N, int M,
                            const JvStats *partial, int n_partial, void *prep_ws, int64_t *out,
                            uint32_t *status, hipStream_t stream);
int jv_compact_max_k();

} // namespace tmamd
