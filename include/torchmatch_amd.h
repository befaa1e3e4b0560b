/*
 * torchmatch_amd.h -- C ABI of the MI355X (gfx950) solver library
 * libtorchmatch_amd.so.
 *
 * Plain pointers and sizes only: every tensor argument is a device pointer
 * to contiguous row-major data, every size is an element count, and every
 * call is stream-ordered on the hipStream_t it is given (0 = null stream).
 * Nothing here allocates, frees or synchronises unless its comment says so.
 * Return values are TM_* codes below; kernels never raise.
 *
 * Reference interfaces replaced (paths relative to the torchmatch
 * repository root):
 *   tm_jv_dense_batch_f32   sources/torchmatch/assignment/cuda/dispatch.cu:137-177
 *                           (jonker_dense_batch_cuda) together with
 *                           assignment/cuda/cuda_common.cuh:215-284
 *                           (compute_inf_sentinel, rewrite_inf_to_sentinel);
 *                           results follow the CPU op
 *                           assignment/cpu/ops.cpp:176-289 bit for bit.
 *   tm_jv_compact_batch_f32 the CPU op assignment::jonker_compact_batch
 *                           (assignment/cpu/ops.cpp:431-433 with
 *                           jonker_compact_core.h:20-301), which has no
 *                           device counterpart in the reference; results
 *                           follow it bit for bit.
 *   tm_jv_unpack_i64        the unpack loop of solve_batch_unpacked,
 *                           assignment/cpu/ops.cpp:291-417 (the device side of
 *                           assignment::jonker_dense_batch_unpacked), which
 *                           assignment/_solve.py:124-164 restates in torch.
 *   tm_sinkhorn_prepare_f32 transport/matrix/_validate.py:58-63,108-110,149-156
 *                           (validate_cost's NaN / -inf checks, the marginal
 *                           sign checks, fuse_mask_into_cost),
 *                           transport/matrix/_schedule.py:68-69 (largest
 *                           finite cost) and _log_sinkhorn.py:36-46
 *                           (_inf_row_col_masks), fused into one pass.
 *   tm_sinkhorn_read_stats  the host readbacks (`.any()`, `.item()`) of
 *                           those checks, one synchronisation for all.
 *   tm_sinkhorn_iterate_f32 sources/torchmatch/transport/matrix/_log_sinkhorn.py:136-221
 *   tm_sinkhorn_f32         (log_sinkhorn_plan) and
 *   tm_sinkhorn_f64         transport/matrix/_unbalanced_sinkhorn.py:30-103
 *                           (unbalanced_sinkhorn_plan); the f64 entry for
 *                           float64 costs, which the reference iterates in
 *                           float64.
 */
#ifndef TORCHMATCH_AMD_H
#define TORCHMATCH_AMD_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Return codes. */
enum {
    TM_OK = 0,
    TM_ERR_INVALID_ARGUMENT = 1, /* negative size, null pointer, bad scalar */
    TM_ERR_UNSUPPORTED_SHAPE = 2,/* shape beyond what the kernels handle */
    TM_ERR_WORKSPACE = 3,        /* workspace missing or too small */
    TM_ERR_LAUNCH = 4,           /* a kernel launch failed (hipGetLastError) */
    TM_ERR_NAN = 5,              /* input holds NaN (reported by tm_jv_check_status) */
    TM_ERR_NEG_INF = 6,          /* input holds -inf (reported by tm_jv_check_status) */
    TM_ERR_HIP = 7,              /* a HIP runtime call failed */
    TM_ERR_INTERNAL = 8          /* a kernel's iteration guard tripped (a bug) */
};

/* Status word bits written by tm_jv_dense_batch_f32 into *d_status. */
enum {
    TM_JV_FLAG_NAN = 1u,
    TM_JV_FLAG_NEG_INF = 2u,
    TM_JV_FLAG_POS_INF = 4u,
    TM_JV_FLAG_ANY_FINITE = 8u,
    TM_JV_FLAG_NEG_ZERO = 16u,  /* input holds -0.0 (informational) */
    /* Set in word [0] by the last write of a K <= 64, B <= 2048 launch whose
     * problems are all solved before its finishing workgroup ends (none holds
     * +inf): every output and both status words are then final, so a caller
     * that cleared word [0] before the launch may poll host-mapped status
     * words for this bit instead of synchronising the stream.  Launches that
     * do not set it are waited for by synchronising the stream. */
    TM_JV_FLAG_DONE = 0x80000000u
};

/* ---- batched Jonker-Volgenant (assignment::jonker_dense_batch) -------- */

/* Largest K = max(N, M) tm_jv_dense_batch_f32 accepts. */
int32_t tm_jv_max_k(void);

/* Device workspace tm_jv_dense_batch_f32 needs for a (B, N, M) batch. */
size_t tm_jv_workspace_bytes(int64_t B, int32_t N, int32_t M);

/* Workspace with which K = max(N, M) > 64 batches also take the prefill: the
 * column reduction and every row's cache of the augmenting row reduction
 * computed by many-wave launches before the solve, which then spends its
 * sequential steps on the reference order alone (C3, 64 x 512 x 768: about
 * 2.6 MB).  Equal to tm_jv_workspace_bytes for K <= 64.  Any workspace of
 * at least tm_jv_workspace_bytes is accepted; the result is the same, bit
 * for bit, with or without the prefill.  No counterpart in the reference:
 * its CPU op keeps thread-local scratch (ops.cpp:246-251). */
size_t tm_jv_workspace_bytes_prefill(int64_t B, int32_t N, int32_t M);

/* Solve B independent (N, M) float32 assignment problems.
 *   costs      device, (B, N, M) contiguous; +inf marks a forbidden pair
 *   out        device, (B, N) int64: row -> column, -1 for rows matched into
 *              padding columns (N > M); identical to the reference CPU op
 *   workspace  device, >= tm_jv_workspace_bytes(B, N, M), any contents
 *   d_status   two uint32 the kernels write with plain stores: device
 *              memory, or the device address of host-mapped pinned memory
 *              (hipHostGetDevicePointer), which saves the copy-back; [0]
 *              receives TM_JV_FLAG_* for the whole batch, [1] is non-zero if
 *              a solve hit its iteration guard
 * The +inf sentinel (max finite + 1) * (K + 1) is computed on the device over
 * the whole batch, as the reference does; no host round trip happens inside.
 * If the batch holds NaN or -inf, `out` is filled with -1 and the flag is set:
 * call tm_jv_check_status to turn the flags into TM_ERR_NAN / TM_ERR_NEG_INF.
 * B == 0, N == 0 or M == 0 launches nothing (the caller fills -1). */
int tm_jv_dense_batch_f32(const float *costs, int64_t B, int32_t N, int32_t M, int64_t *out,
                          void *workspace, size_t workspace_bytes, uint32_t *d_status,
                          hipStream_t stream);

/* tm_jv_dense_batch_f32, then the wait for its result, in one call: returns
 * once every output is final for work that follows on `stream`, with the
 * batch's status decoded (TM_OK, TM_ERR_NAN, TM_ERR_NEG_INF, TM_ERR_INTERNAL,
 * or a launch / HIP error); the replacement for the reference's launch plus
 * its status readback (dispatch.cu:137-177, cuda_common.cuh:241-249).  For
 * K <= 64 and B <= 2048 every solve workgroup also writes its problem's
 * summary to pinned host memory the library holds per host thread and
 * device, and the host folds those as they arrive, so a batch with no +inf,
 * NaN or -inf returns without a second launch or a stream synchronisation.
 * That memory (8,200 bytes per block) is the one allocation these entry
 * points make: a block is taken from a per-device pool at a thread's first
 * call on a device (allocated only when the pool is empty) and returned to
 * the pool when the thread exits, so the process holds one block per device
 * for each host thread that has called and is alive at once, and keeps the
 * blocks until it ends.
 * `replays` (host, may be NULL) receives the number of problems that left
 * the certified path for the exact replay on that path (0 otherwise).  Calls
 * on one host thread must not overlap (each returns before the next starts).
 * Same arguments, workspace and results as tm_jv_dense_batch_f32; no status
 * words are passed. */
int tm_jv_dense_batch_f32_sync(const float *costs, int64_t B, int32_t N, int32_t M,
                               int64_t *out, void *workspace, size_t workspace_bytes,
                               uint32_t *replays, hipStream_t stream);

/* The same for tm_jv_compact_batch_f32. */
int tm_jv_compact_batch_f32_sync(const float *costs, int64_t B, int32_t N, int32_t M,
                                 int64_t *out, void *workspace, size_t workspace_bytes,
                                 uint32_t *replays, hipStream_t stream);

/* tm_jv_dense_batch_f32 without a workspace argument and without any device
 * allocation.  No counterpart in the reference: it is for callers that cannot
 * allocate (code under graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The workspace is a fixed device array inside the
 * library, tm_jv_noalloc_scratch_bytes() bytes per GPU (35,072), held from the
 * library's load until the process ends; its address is looked up once per
 * device on the first call for that device.  Calls that overlap on one GPU
 * share the array and race: order them (one stream, or events).  Arguments,
 * status words, results and error codes as tm_jv_dense_batch_f32;
 * TM_ERR_WORKSPACE if a shape would need more than the array holds (none
 * does: tm_jv_workspace_bytes never exceeds it). */
int tm_jv_dense_batch_f32_noalloc(const float *costs, int64_t B, int32_t N, int32_t M,
                                  int64_t *out, uint32_t *d_status, hipStream_t stream);

/* Size of the fixed device workspace tm_jv_dense_batch_f32_noalloc uses. */
size_t tm_jv_noalloc_scratch_bytes(void);

/* Largest K = max(N, M) tm_jv_compact_batch_f32 accepts. */
int32_t tm_jv_compact_max_k(void);

/* Solve B problems like tm_jv_dense_batch_f32 (same arguments, workspace,
 * status words and sentinel / padding rules) with the solver of
 * assignment::jonker_compact_batch instead: out is identical to that CPU op's
 * mapping, whose tie rules differ from the dense solver's. */
int tm_jv_compact_batch_f32(const float *costs, int64_t B, int32_t N, int32_t M, int64_t *out,
                            void *workspace, size_t workspace_bytes, uint32_t *d_status,
                            hipStream_t stream);

/* Problems of the last tm_jv_dense_batch_f32 / tm_jv_compact_batch_f32 call on
 * `workspace` (K <= 64) whose certified shortest-path solve did not prove a
 * unique optimum and that were solved again by the exact replay of the
 * reference's order (ties, near-ties).  Copies one word to *count and
 * synchronises `stream`.  A diagnostic with no counterpart in the reference.
 * TORCHMATCH_AMD_JV_CERTIFY=0 in the environment switches the certified path
 * off (every problem replays). */
int tm_jv_read_replays(const void *workspace, uint32_t *count, hipStream_t stream);

/* Copy the two status words to the host and synchronise `stream` (the only
 * host sync of the JV path, mirroring the reference's validation readback,
 * cuda_common.cuh:241-249).  Returns TM_OK, TM_ERR_NAN, TM_ERR_NEG_INF,
 * TM_ERR_INTERNAL or TM_ERR_HIP. */
int tm_jv_check_status(const uint32_t *d_status, hipStream_t stream);

/* The same verdict from status words already on the host (host-mapped
 * d_status after the caller synchronised the stream).  No HIP call. */
int tm_jv_status_code(const uint32_t *h_status);

/* Unpack B packed mappings (the `out` of tm_jv_dense_batch_f32: row -> column
 * in [0, M) or -1) into the tuple of assignment::jonker_dense_batch_unpacked:
 *   matches         device, (B, N, 2) int64: (row, col) of matched rows in row
 *                   order, -1 after n_matches[b] pairs
 *   unmatched_rows  device, (B, N) int64: unmatched rows, increasing, then -1
 *   unmatched_cols  device, (B, M) int64: columns no row took, increasing,
 *                   then -1
 *   n_matches       device, (B,) int64
 * Same contents as the reference CPU op (ops.cpp:387-414, -1 padding as its
 * at::full(-1) leaves).  M <= 4096. */
int tm_jv_unpack_i64(const int64_t *packed, int64_t B, int32_t N, int32_t M, int64_t *matches,
                     int64_t *unmatched_rows, int64_t *unmatched_cols, int64_t *n_matches,
                     hipStream_t stream);

/* ---- log-domain Sinkhorn (transport::log_sinkhorn / unbalanced_sinkhorn) */

/* Flag bits tm_sinkhorn_read_stats reports. */
enum {
    TM_SK_FLAG_NAN = 1u,          /* the cost holds NaN (before the mask) */
    TM_SK_FLAG_NEG_INF = 2u,      /* the cost holds -inf (before the mask) */
    TM_SK_FLAG_A_NEG = 4u,        /* a holds a negative entry */
    TM_SK_FLAG_B_NEG = 8u,        /* b holds a negative entry */
    TM_SK_FLAG_ANY_FINITE = 16u   /* the masked cost holds a finite entry */
};

/* Device workspace the Sinkhorn calls below need.  The size depends on the
 * step form chosen for the shape (TORCHMATCH_AMD_SINKHORN_FUSED); keep that
 * variable unchanged between this query and the calls that use the
 * workspace (a smaller workspace is refused with TM_ERR_WORKSPACE). */
size_t tm_sinkhorn_workspace_bytes(int64_t B, int64_t N, int64_t M);

/* First half of a solve: one pass over the (B, N, M) float32 cost and the
 * marginals, all on `stream`, no host synchronisation.
 *   cost       device (B, N, M); +inf = forbidden pair
 *   keep       device (B, N, M) bytes or NULL: pairs with keep == 0 are
 *              forbidden (the cost is read as +inf there), i.e. the
 *              reference's fuse_mask_into_cost (transport/matrix/
 *              _validate.py:149-156) without materialising the fused cost
 *   a, b       device marginals (B, N) and (B, M)
 *   k_eps      > 0: also write the log kernel -C/k_eps into the workspace
 *              (pass the same value to tm_sinkhorn_iterate_f32); 0: do not
 * The pass also records what the reference's validation and schedule read
 * from the cost (transport/matrix/_validate.py:58-63, 108-110 and
 * _schedule.py:68-69): NaN / -inf in the cost, negative marginal entries and
 * the largest finite (masked) cost.  tm_sinkhorn_read_stats fetches them. */
int tm_sinkhorn_prepare_f32(const float *cost, const uint8_t *keep, const float *a,
                            const float *b, int64_t B, int64_t N, int64_t M, float k_eps,
                            void *workspace, size_t workspace_bytes, hipStream_t stream);

/* Copy the statistics of the last tm_sinkhorn_prepare_f32 on `workspace` to
 * the host and synchronise `stream` (the only host sync of a solve).
 * *flags receives TM_SK_FLAG_* bits, *max_finite the largest finite masked
 * cost (-inf when TM_SK_FLAG_ANY_FINITE is clear). */
int tm_sinkhorn_read_stats(const void *workspace, int64_t B, int64_t N, int64_t M,
                           uint32_t *flags, float *max_finite, hipStream_t stream);

/* Second half: the log-domain Sinkhorn iteration of the reference over the
 * workspace tm_sinkhorn_prepare_f32 filled (same cost, keep, B, N, M), and
 * the log transport plan.
 *   eps_sched  HOST array of n_iter float64 epsilons (the reference schedule)
 *   rho        <= 0: balanced (log_sinkhorn); > 0: unbalanced with KL
 *              penalty rho (damping 1 / (1 + eps / rho) per step)
 *   k_eps      the k_eps given to tm_sinkhorn_prepare_f32
 *   log_plan   device (B, N, M) output, may be NULL to skip the plan
 *   log_u, log_v  device (B, N), (B, M) outputs: the final scaling
 *              potentials (f = -eps * log_u, g = -eps * log_v)
 * With B >= 2 the steps of part of the batch run on a side stream of the
 * library's own (created on the first such call per device of `stream`,
 * default priority), forked from and joined back into `stream` with events:
 * the call stays stream-ordered on `stream`.  TORCHMATCH_AMD_SINKHORN_GROUPS=1
 * keeps every launch on `stream`, and so does a `stream` under graph capture.
 * Threading: calls from several host threads, on the same or different
 * streams, are safe; each call holds a per-device lock from its fork to its
 * join, so the side streams never serve two callers' segments interleaved.
 * Calls that share a workspace must be ordered by the caller. */
int tm_sinkhorn_iterate_f32(const float *cost, const uint8_t *keep, int64_t B, int64_t N,
                            int64_t M, const double *eps_sched, int32_t n_iter, double rho,
                            float k_eps, float *log_plan, float *log_u, float *log_v,
                            void *workspace, size_t workspace_bytes, hipStream_t stream);

/* Both halves without a mask and without reading the statistics back: the
 * cost must hold no NaN / -inf and the marginals must be non-negative.
 *   a, b       device marginals (B, N) and (B, M)
 *   other arguments as tm_sinkhorn_iterate_f32 */
int tm_sinkhorn_f32(const float *cost, const float *a, const float *b, int64_t B, int64_t N,
                    int64_t M, const double *eps_sched, int32_t n_iter, double rho,
                    float *log_plan, float *log_u, float *log_v, void *workspace,
                    size_t workspace_bytes, hipStream_t stream);

/* ---- float64 Sinkhorn ---------------------------------------------------
 * The reference iterates in the cost's dtype (transport/matrix/
 * _log_sinkhorn.py:184,191, _unbalanced_sinkhorn.py:60,67): a float64 cost
 * is solved in float64, with the same recurrence, shift rule, keep-previous
 * rule, damping and plan expression as tm_sinkhorn_iterate_f32.  The caller
 * validates the cost (no NaN / -inf), fuses any mask into it (+inf) and
 * builds the schedule; nothing is read back.
 *   cost, a, b, log_plan, log_u, log_v  device float64 tensors of the shapes
 *   and meanings of tm_sinkhorn_f32; log_plan may be NULL
 *   workspace  device, >= tm_sinkhorn_f64_workspace_bytes(B, N, M)
 * Any B: every launch strides its grid over the batch. */
size_t tm_sinkhorn_f64_workspace_bytes(int64_t B, int64_t N, int64_t M);
int tm_sinkhorn_f64(const double *cost, const double *a, const double *b, int64_t B,
                    int64_t N, int64_t M, const double *eps_sched, int32_t n_iter, double rho,
                    double *log_plan, double *log_u, double *log_v, void *workspace,
                    size_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TORCHMATCH_AMD_H */
