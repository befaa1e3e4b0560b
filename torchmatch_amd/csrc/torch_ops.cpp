// torch_ops.cpp -- torch dispatcher registrations over the C ABI.
//
// Only CUDA-key kernels live here (ROCm tensors have device type "cuda").
// The schema of `assignment::jonker_dense_batch` belongs to whoever defines
// the `assignment` library (the reference CPU extension, ops.cpp:486-495, or
// torchmatch_amd/_loader.py when that extension is absent); this file adds
// the device kernel exactly where the reference's CUDA extension adds its own
// (assignment/cuda/dispatch.cu:181-186).
//
// The private `torchmatch_amd::sinkhorn_prepare` / `sinkhorn_iterate` ops are
// what the Python custom ops `transport::log_sinkhorn`,
// `transport::unbalanced_sinkhorn` and `transport::sinkhorn_divergence` call
// for device tensors.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <vector>

#include "../../include/torchmatch_amd.h"

namespace {

hipStream_t current_stream(const at::Tensor &t) {
    return c10::hip::getCurrentHIPStream(t.get_device()).stream();
}

// Mirrors check_not_capturing (assignment/cuda/dispatch.cu:97-106): the op
// reads its validation flags back to the host, which stream capture forbids.
void check_not_capturing(hipStream_t stream, const char *op_name) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    const hipError_t e = hipStreamIsCapturing(stream, &status);
    TORCH_CHECK(e == hipSuccess, op_name, ": hipStreamIsCapturing failed: ",
                hipGetErrorString(e));
    TORCH_CHECK(status == hipStreamCaptureStatusNone, op_name,
                " performs a host-side synchronization and cannot run inside CUDA graph "
                "capture (e.g. torch.compile(mode=\"reduce-overhead\")); call it outside the "
                "captured region.");
}

void check_rc(int rc, const char *op_name) {
    switch (rc) {
    case TM_OK:
        return;
    case TM_ERR_NAN:
        TORCH_CHECK(false, "cost matrix contains NaN; use +inf for forbidden pairs, NaN "
                           "signals an upstream bug");
    case TM_ERR_NEG_INF:
        TORCH_CHECK(false, "cost matrix contains -inf; -inf has no forbidden-edge meaning");
    case TM_ERR_UNSUPPORTED_SHAPE:
        TORCH_CHECK(false, op_name, ": shape not supported by the gfx950 kernels");
    case TM_ERR_INVALID_ARGUMENT:
        TORCH_CHECK(false, op_name, ": invalid argument");
    case TM_ERR_WORKSPACE:
        TORCH_CHECK(false, op_name, ": workspace too small");
    case TM_ERR_INTERNAL:
        TORCH_CHECK(false, op_name, ": internal error (iteration guard tripped)");
    case TM_ERR_LAUNCH:
        TORCH_CHECK(false, op_name, ": kernel launch failed: ",
                    hipGetErrorString(hipGetLastError()));
    default:
        TORCH_CHECK(false, op_name, ": HIP runtime error (code ", rc, ")");
    }
}

using JvSolver = int (*)(const float *, int64_t, int32_t, int32_t, int64_t *, void *, size_t,
                        uint32_t *, hipStream_t);

// Shared body of the batched JV ops: checks, float32 view, workspace, then
// the library's synchronous solve (launch, wait, status).
at::Tensor jv_batch_hip(const at::Tensor &costs, JvSolver solver, int64_t max_k,
                        const char *op_name) {
    TORCH_CHECK(costs.is_cuda(), "costs must be a CUDA tensor");
    TORCH_CHECK(costs.dim() == 3, "costs must be 3D (B, N, M), got ", costs.dim());
    TORCH_CHECK(costs.scalar_type() == at::kFloat || costs.scalar_type() == at::kDouble,
                "costs must be float32 or float64, got ", costs.scalar_type());
    TORCH_CHECK(costs.is_contiguous(), "costs must be contiguous");
    const c10::DeviceGuard guard(costs.device());

    const int64_t B = costs.size(0);
    const int64_t N = costs.size(1);
    const int64_t M = costs.size(2);
    auto out = at::empty({B, N}, costs.options().dtype(at::kLong));
    if (B == 0 || N == 0 || M == 0) {
        out.fill_(-1);
        return out;
    }
    const int64_t K = N > M ? N : M;
    TORCH_CHECK(K <= max_k, op_name, " (gfx950) supports K = max(N, M) <= ", max_k, ", got K=",
                K);

    const hipStream_t stream = current_stream(costs);
    check_not_capturing(stream, op_name);

    // float64 input is solved in float32, as the reference device op does
    // (dispatch.cu:156).
    const at::Tensor cf = costs.scalar_type() == at::kFloat ? costs : costs.to(at::kFloat);
    // K > 64: with room for the prefill (column reduction and row caches)
    const size_t ws_bytes = tm_jv_workspace_bytes_prefill(B, (int32_t)N, (int32_t)M);
    auto ws = at::empty({(int64_t)ws_bytes}, costs.options().dtype(at::kByte));
    // launch, wait and status in one call (the library folds the batch's
    // status on the host as the solve publishes it)
    const int rc = solver(cf.data_ptr<float>(), B, (int32_t)N, (int32_t)M,
                          out.data_ptr<int64_t>(), ws.data_ptr(), ws_bytes, nullptr, stream);
    check_rc(rc, op_name);
    return out;
}

// The device unpack (tm_jv_unpack_i64) of a packed (B, N) mapping into the
// tuple the reference CPU ops return (assignment/cpu/ops.cpp:291-417).
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor>
unpack_hip(const at::Tensor &costs, const at::Tensor &packed, const char *op_name) {
    const c10::DeviceGuard guard(costs.device());
    const int64_t B = costs.size(0), N = costs.size(1), M = costs.size(2);
    const auto lopts = costs.options().dtype(at::kLong);
    auto matches = at::empty({B, N, 2}, lopts);
    auto ur = at::empty({B, N}, lopts);
    auto uc = at::empty({B, M}, lopts);
    auto nm = at::zeros({B}, lopts);
    if (B == 0 || N == 0 || M == 0) {
        // the CPU op's empty-shape return (ops.cpp:310-316)
        return {matches, ur, uc, nm};
    }
    const int rc = tm_jv_unpack_i64(packed.data_ptr<int64_t>(), B, (int32_t)N, (int32_t)M,
                                    matches.data_ptr<int64_t>(), ur.data_ptr<int64_t>(),
                                    uc.data_ptr<int64_t>(), nm.data_ptr<int64_t>(),
                                    current_stream(costs));
    check_rc(rc, op_name);
    return {matches, ur, uc, nm};
}

// CUDA-key kernel of assignment::jonker_dense_batch.
// Reference: assignment/cuda/dispatch.cu:137-177; results follow the CPU op
// assignment/cpu/ops.cpp:176-289 (rectangular input accepted, like the CPU op).
at::Tensor jonker_dense_batch_hip(const at::Tensor &costs) {
    return jv_batch_hip(costs, &tm_jv_dense_batch_f32_sync, tm_jv_max_k(), "jonker_dense_batch");
}

// CUDA-key kernel of assignment::jonker_dense_batch_unpacked (CPU op at
// assignment/cpu/ops.cpp:436-440, registered at :504).
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor>
jonker_dense_batch_unpacked_hip(const at::Tensor &costs) {
    return unpack_hip(costs, jonker_dense_batch_hip(costs), "jonker_dense_batch_unpacked");
}

// CUDA-key kernel of assignment::jonker_compact_batch: the mapping of the CPU
// op assignment/cpu/ops.cpp:431-433 (solve_batch around the compact solver of
// jonker_compact_core.h), which has no device counterpart in the reference.
at::Tensor jonker_compact_batch_hip(const at::Tensor &costs) {
    return jv_batch_hip(costs, &tm_jv_compact_batch_f32_sync, tm_jv_compact_max_k(),
                        "jonker_compact_batch");
}

// CUDA-key kernel of assignment::jonker_compact_batch_unpacked (CPU op at
// assignment/cpu/ops.cpp:441-445).
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor>
jonker_compact_batch_unpacked_hip(const at::Tensor &costs) {
    return unpack_hip(costs, jonker_compact_batch_hip(costs), "jonker_compact_batch_unpacked");
}

void check_keep(const at::Tensor &cost, const c10::optional<at::Tensor> &keep) {
    if (!keep.has_value())
        return;
    TORCH_CHECK(keep->is_cuda() && keep->device() == cost.device(),
                "sinkhorn: keep must be on the cost's device");
    TORCH_CHECK(keep->scalar_type() == at::kBool, "sinkhorn: keep must be a bool tensor");
    TORCH_CHECK(keep->sizes() == cost.sizes() && keep->is_contiguous(),
                "sinkhorn: keep must be contiguous with the cost's shape");
}

const uint8_t *keep_ptr(const c10::optional<at::Tensor> &keep) {
    return keep.has_value() ? reinterpret_cast<const uint8_t *>(keep->data_ptr<bool>()) : nullptr;
}

// torchmatch_amd::sinkhorn_prepare -- the one pass over cost, keep mask and
// marginals that a device Sinkhorn solve starts with.  Returns the workspace
// (device bytes, handed to sinkhorn_iterate) and, when read_stats, a CPU
// float64 tensor (flags, largest finite masked cost) read back with one
// synchronisation; an empty tensor otherwise.
std::tuple<at::Tensor, at::Tensor>
sinkhorn_prepare_hip(const at::Tensor &cost, const c10::optional<at::Tensor> &keep,
                     const at::Tensor &a, const at::Tensor &b, double k_eps, bool read_stats) {
    TORCH_CHECK(cost.is_cuda() && a.is_cuda() && b.is_cuda(),
                "sinkhorn: cost, a and b must be CUDA tensors");
    TORCH_CHECK(cost.dim() == 3, "sinkhorn: cost must be 3D (B, N, M)");
    TORCH_CHECK(cost.scalar_type() == at::kFloat && a.scalar_type() == at::kFloat &&
                    b.scalar_type() == at::kFloat,
                "sinkhorn: the gfx950 kernels compute in float32");
    TORCH_CHECK(cost.is_contiguous() && a.is_contiguous() && b.is_contiguous(),
                "sinkhorn: cost, a and b must be contiguous");
    const int64_t B = cost.size(0), N = cost.size(1), M = cost.size(2);
    TORCH_CHECK(a.dim() == 2 && a.size(0) == B && a.size(1) == N, "sinkhorn: a must be (B, N)");
    TORCH_CHECK(b.dim() == 2 && b.size(0) == B && b.size(1) == M, "sinkhorn: b must be (B, M)");
    check_keep(cost, keep);
    const c10::DeviceGuard guard(cost.device());
    const size_t ws_bytes = tm_sinkhorn_workspace_bytes(B, N, M);
    auto ws = at::empty({(int64_t)ws_bytes}, cost.options().dtype(at::kByte));
    const hipStream_t stream = current_stream(cost);
    if (read_stats)
        check_not_capturing(stream, "the transport Sinkhorn input check");
    int rc = tm_sinkhorn_prepare_f32(cost.data_ptr<float>(), keep_ptr(keep), a.data_ptr<float>(),
                                     b.data_ptr<float>(), B, N, M, (float)k_eps, ws.data_ptr(),
                                     ws_bytes, stream);
    check_rc(rc, "sinkhorn_prepare");
    at::Tensor stats = at::empty({0}, at::TensorOptions().dtype(at::kDouble));
    if (read_stats) {
        uint32_t flags = 0;
        float max_finite = 0.f;
        rc = tm_sinkhorn_read_stats(ws.data_ptr(), B, N, M, &flags, &max_finite, stream);
        TORCH_CHECK(rc == TM_OK, "sinkhorn_prepare: reading the statistics back failed: ",
                    hipGetErrorString(hipGetLastError()));
        stats = at::empty({2}, at::TensorOptions().dtype(at::kDouble));
        stats.data_ptr<double>()[0] = (double)flags;
        stats.data_ptr<double>()[1] = (double)max_finite;
    }
    return {ws, stats};
}

// torchmatch_amd::sinkhorn_iterate -- device Sinkhorn over a precomputed
// epsilon schedule on a workspace from sinkhorn_prepare (same cost and keep).
// Returns (log_plan, log_u, log_v); log_plan is empty when write_plan is false.
std::tuple<at::Tensor, at::Tensor, at::Tensor>
sinkhorn_iterate_hip(const at::Tensor &cost, const c10::optional<at::Tensor> &keep,
                     const at::Tensor &ws, at::ArrayRef<double> eps_sched, double rho,
                     double k_eps, bool write_plan) {
    TORCH_CHECK(cost.is_cuda() && ws.is_cuda(), "sinkhorn: cost and workspace must be CUDA tensors");
    TORCH_CHECK(cost.dim() == 3 && cost.scalar_type() == at::kFloat && cost.is_contiguous(),
                "sinkhorn: cost must be a contiguous float32 (B, N, M) tensor");
    TORCH_CHECK(!eps_sched.empty(), "sinkhorn: empty epsilon schedule");
    check_keep(cost, keep);
    const int64_t B = cost.size(0), N = cost.size(1), M = cost.size(2);
    const c10::DeviceGuard guard(cost.device());
    auto log_u = at::empty({B, N}, cost.options());
    auto log_v = at::empty({B, M}, cost.options());
    at::Tensor log_plan = write_plan ? at::empty({B, N, M}, cost.options())
                                     : at::empty({0}, cost.options());
    if (B == 0)
        return {log_plan, log_u, log_v};
    const int rc = tm_sinkhorn_iterate_f32(
        cost.data_ptr<float>(), keep_ptr(keep), B, N, M, eps_sched.data(),
        (int32_t)eps_sched.size(), rho, (float)k_eps,
        write_plan ? log_plan.data_ptr<float>() : nullptr, log_u.data_ptr<float>(),
        log_v.data_ptr<float>(), ws.data_ptr(), (size_t)ws.numel(), current_stream(cost));
    check_rc(rc, "sinkhorn_iterate");
    return {log_plan, log_u, log_v};
}

// torchmatch_amd::sinkhorn_f64 -- the whole float64 solve (the reference
// iterates in the cost's dtype) on a cost already validated and mask-fused by
// the caller.  Returns (log_plan, log_u, log_v); log_plan is empty when
// write_plan is false.
std::tuple<at::Tensor, at::Tensor, at::Tensor>
sinkhorn_f64_hip(const at::Tensor &cost, const at::Tensor &a, const at::Tensor &b,
                 at::ArrayRef<double> eps_sched, double rho, bool write_plan) {
    TORCH_CHECK(cost.is_cuda() && a.is_cuda() && b.is_cuda(),
                "sinkhorn: cost, a and b must be CUDA tensors");
    TORCH_CHECK(cost.dim() == 3 && cost.scalar_type() == at::kDouble && cost.is_contiguous(),
                "sinkhorn: cost must be a contiguous float64 (B, N, M) tensor");
    TORCH_CHECK(a.scalar_type() == at::kDouble && b.scalar_type() == at::kDouble &&
                    a.is_contiguous() && b.is_contiguous(),
                "sinkhorn: a and b must be contiguous float64 tensors");
    TORCH_CHECK(!eps_sched.empty(), "sinkhorn: empty epsilon schedule");
    const int64_t B = cost.size(0), N = cost.size(1), M = cost.size(2);
    TORCH_CHECK(a.dim() == 2 && a.size(0) == B && a.size(1) == N, "sinkhorn: a must be (B, N)");
    TORCH_CHECK(b.dim() == 2 && b.size(0) == B && b.size(1) == M, "sinkhorn: b must be (B, M)");
    const c10::DeviceGuard guard(cost.device());
    auto log_u = at::empty({B, N}, cost.options());
    auto log_v = at::empty({B, M}, cost.options());
    at::Tensor log_plan = write_plan ? at::empty({B, N, M}, cost.options())
                                     : at::empty({0}, cost.options());
    const size_t ws_bytes = tm_sinkhorn_f64_workspace_bytes(B, N, M);
    auto ws = at::empty({(int64_t)(ws_bytes > 0 ? ws_bytes : 1)}, cost.options().dtype(at::kByte));
    const int rc = tm_sinkhorn_f64(
        cost.data_ptr<double>(), a.data_ptr<double>(), b.data_ptr<double>(), B, N, M,
        eps_sched.data(), (int32_t)eps_sched.size(), rho,
        write_plan ? log_plan.data_ptr<double>() : nullptr, log_u.data_ptr<double>(),
        log_v.data_ptr<double>(), ws.data_ptr(), ws_bytes, current_stream(cost));
    check_rc(rc, "sinkhorn_f64");
    return {log_plan, log_u, log_v};
}

} // namespace

TORCH_LIBRARY_IMPL(assignment, CUDA, m) {
    m.impl("jonker_dense_batch", &jonker_dense_batch_hip);
    m.impl("jonker_dense_batch_unpacked", &jonker_dense_batch_unpacked_hip);
    m.impl("jonker_compact_batch", &jonker_compact_batch_hip);
    m.impl("jonker_compact_batch_unpacked", &jonker_compact_batch_unpacked_hip);
}

TORCH_LIBRARY(torchmatch_amd, m) {
    m.def("sinkhorn_prepare(Tensor cost, Tensor? keep, Tensor a, Tensor b, float k_eps, "
          "bool read_stats) -> (Tensor, Tensor)");
    m.def("sinkhorn_iterate(Tensor cost, Tensor? keep, Tensor ws, float[] eps_sched, "
          "float rho, float k_eps, bool write_plan) -> (Tensor, Tensor, Tensor)");
    m.def("sinkhorn_f64(Tensor cost, Tensor a, Tensor b, float[] eps_sched, float rho, "
          "bool write_plan) -> (Tensor, Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(torchmatch_amd, CUDA, m) {
    m.impl("sinkhorn_prepare", &sinkhorn_prepare_hip);
    m.impl("sinkhorn_iterate", &sinkhorn_iterate_hip);
    m.impl("sinkhorn_f64", &sinkhorn_f64_hip);
}
