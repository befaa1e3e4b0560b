// jv_batch.h -- internal declarations shared by the JV kernels and the C ABI.
#pragma once

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

// Upper bound on the blocks of the statistics pass (and so on the partial
// records every solve workgroup folds).
constexpr int kJvMaxStatBlocks = 256;

struct JvStats {
    float max_finite;
    float min_finite;
    uint32_t flags;
    uint32_t pad;
};

} // namespace tmamd
