/*
 * hm_moe.h -- C ABI of the MI355X (gfx950) MoE-block engine.
 *
 * This is the boundary between the C++20 host layer (HipBackend,
 * HipTensorBackend, HipMoEBlock) and the hand-written HIP kernels in
 * libhm_kernels.so.  It replaces, for the device-resident MoE block, what the
 * reference reaches through its C++ virtual interfaces and its CUDA kernel
 * free functions (SHOnnay/hypermoe-engine):
 *
 *   ComputeBackend            src/backend/Backend.hpp:36-71
 *   TensorBackend             src/tensor/backend/TensorBackend.hpp:11-39
 *   MoERuntime::executeBatch  src/core/runtime/MoERuntime.hpp:57-60
 *   CUDA kernels              src/backend/cuda/CudaKernels.hpp:10-46
 *
 * Conventions
 *   - Every pointer argument is a DEVICE pointer unless its comment says
 *     host.  The caller owns all memory; nothing here allocates device memory
 *     except hm_device_alloc/hm_host_alloc.
 *   - `stream` is a hipStream_t passed as void* (NULL = default stream).
 *     Launchers are asynchronous on that stream and never synchronise.
 *   - Every function returns an hm_status.  HM_ERR_INVALID, HM_ERR_OVERFLOW
 *     and HM_ERR_RUNTIME map to the reference's std::invalid_argument,
 *     std::overflow_error and std::runtime_error.  A HIP failure returns
 *     HM_ERR_RUNTIME and hm_last_hip_error() gives the hipError_t.
 *   - Conditions only the device can see (a non-finite router score, a
 *     softmax/renormalisation failure) are reported through the device
 *     status word `status` (int32, HM_STATUS_* bits), which the caller reads
 *     back; the reference throws std::runtime_error for them
 *     (src/router/CpuRouterBackend.cpp:47,57-59,83-85).  A token whose
 *     softmax or renormalisation failed gets placeholder ids 0..top_k-1 with
 *     zero scores, so that the launches queued after it stay in range.
 *   - No function throws.
 */
#ifndef HM_MOE_H
#define HM_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HM_ABI_VERSION 1

typedef enum hm_status {
    HM_OK = 0,
    HM_ERR_INVALID = 1,   /* std::invalid_argument */
    HM_ERR_OVERFLOW = 2,  /* std::overflow_error   */
    HM_ERR_RUNTIME = 3,   /* std::runtime_error (HIP or launch failure) */
    HM_ERR_UNSUPPORTED = 4
} hm_status;

/* Device status word bits (written by kernels, read by the host). */
#define HM_STATUS_NONFINITE_SCORE 1u   /* CpuRouterBackend.cpp:47        */
#define HM_STATUS_SOFTMAX_FAILED 2u    /* CpuRouterBackend.cpp:57-59     */
#define HM_STATUS_RENORM_FAILED 4u     /* CpuRouterBackend.cpp:83-85     */

/* Routing flags, RouterConfig (src/router/RouterConfig.hpp:22-29). */
#define HM_ROUTE_SOFTMAX 1u  /* RoutingNormalization::Softmax, else None */
#define HM_ROUTE_RENORM 2u   /* renormalizeSelected                       */
/* Execution flag for hm_moe_block_forward: run the INT8 expert GEMMs on the
 * scalar reference kernels instead of MFMA (identical integers and float
 * operation sequence; used to pin the MFMA kernels). */
#define HM_EXEC_GENERIC 0x100u
/* Execution flag for hm_moe_block_forward: INT8 experts always take the
 * integer-limb GEMMs.  Without it a block of at most HM_GEMV_MAX_TOKENS
 * tokens and HM_GEMV_MAX_PAIRS (token, expert) pairs (decode) takes the
 * W8A32 GEMV kernels instead, which stream each selected expert's weights
 * once and compute in FP32 (within 1e-4 of the reference, not bit-identical
 * to the limb arithmetic); larger blocks, decode ones included, take the
 * limb GEMMs. */
#define HM_EXEC_LIMBS 0x200u
#define HM_GEMV_MAX_TOKENS 16
#define HM_GEMV_MAX_PAIRS 64
/* Execution flag for hm_router_topk / hm_moe_block_forward: every router
 * logit is computed with the reference's sequential FP64 chain instead of
 * certifying the parallel sums (the results are identical; the flag
 * exercises the fallback). */
#define HM_EXEC_ROUTE_SEQUENTIAL 0x400u
/* Execution flag for hm_moe_block_forward: INT8 prefill experts with at most
 * 32 grouped rows take the bounded split-K GEMM (K split over a workgroup's
 * waves, exact integer partials; the same bits as without it) instead of
 * the tile GEMMs' partial tiles.  Off by default: on this GPU it is slower
 * at every batch size measured (the tiles stream the same weights faster). */
#define HM_EXEC_SPLIT_K 0x800u

/* Expert weight dtypes (src/tensor/DType.hpp:9-14 numbering). */
#define HM_DTYPE_FP32 0
#define HM_DTYPE_INT8 3

int hm_abi_version(void);
const char* hm_status_string(int status);
/* Last hipError_t seen by a launcher on this host thread (0 = none). */
int hm_last_hip_error(void);

/* ---- Device runtime (ComputeBackend surface, src/backend/Backend.hpp:36-71) */
int hm_device_count(int* count_out /* host */);
int hm_set_device(int ordinal);
int hm_device_alloc(void** ptr_out /* host */, size_t bytes);
int hm_device_free(void* ptr);
int hm_host_alloc(void** ptr_out /* host */, size_t bytes); /* pinned */
int hm_host_free(void* ptr);
int hm_memcpy_h2d(void* dst, const void* src_host, size_t bytes, void* stream);
int hm_memcpy_d2h(void* dst_host, const void* src, size_t bytes, void* stream);
int hm_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
int hm_stream_create(void** stream_out /* host */);
int hm_stream_destroy(void* stream);
int hm_stream_synchronize(void* stream);
int hm_event_create(void** event_out /* host */);
int hm_event_destroy(void* event);
int hm_event_record(void* event, void* stream);
int hm_event_synchronize(void* event);
int hm_stream_wait_event(void* stream, void* event);
int hm_event_elapsed_ms(float* ms_out /* host */, void* start, void* stop);
int hm_mem_info(size_t* free_out /* host */, size_t* total_out /* host */);

/* ---- A1  RMSNorm (src/transformer/norm/RMSNorm.cpp:65-77) ----------------
 * y[r,i] = float(double(x[r,i]) * inv_r * double(gamma[i])),
 * inv_r = 1/sqrt(sum_i double(x)^2 / width + double(eps)), the sum taken in
 * ascending i exactly as the reference's sequential loop.  Bit-exact. */
int hm_rmsnorm(const float* x, const float* gamma, float* y, int64_t rows,
               int64_t width, float eps, void* stream);

/* ---- A2  Router (src/router/CpuRouterBackend.cpp:35-91) -----------------
 * logits[t,e] = float(sum_k double(h[t,k]) * double(w[k,e])), k ascending;
 * softmax with glibc-expf-exact float exp and double denominator; top-k by
 * (score desc, expert id asc); optional renormalisation by the double sum of
 * the selected scores in rank order.  ids/scores are [tokens x top_k] in
 * rank order.  Bit-exact.  The logits go to logits_out, or, when it is NULL,
 * to `route_ws` (hm_route_workspace_bytes(tokens, hidden, experts) bytes, 16-byte
 * aligned).  With route_ws given, the logit sums take a certified parallel
 * form whose partials live in route_ws: FP64 block chains for batches of at
 * most 16 tokens, FP64 matrix-core sums for larger batches when E % 64 == 0
 * and H % 16 == 0.  A logit whose float the error bound does not settle is
 * recomputed by the sequential chain, so the results are those of the
 * sequential form.  `flags`: HM_ROUTE_* bits, optionally
 * HM_EXEC_ROUTE_SEQUENTIAL. */
size_t hm_route_workspace_bytes(int64_t tokens, int64_t hidden, int64_t experts);
int hm_router_topk(const float* h, const float* w, int64_t tokens,
                   int64_t hidden, int64_t experts, int32_t top_k,
                   uint32_t flags, uint32_t* ids, float* scores,
                   float* logits_out, int32_t* status, void* route_ws,
                   void* stream);

/* ---- A3  Token permute (src/router/CpuRouterBackend.cpp:140-159) ---------
 * Stable counting sort of the tokens*top_k (token, rank) pairs by expert id:
 * counts[E], offsets[E+1], perm_tokens/perm_weights[tokens*top_k] in group
 * order (groups by ascending expert id, tokens ascending inside a group),
 * slots[tokens*top_k]: the grouped row of pair (t, r).  Bit-exact.  No
 * global atomics: per-chunk LDS histograms, then each chunk ranks its pairs.
 * `workspace`: hm_permute_workspace_bytes(...) bytes (may be NULL when that
 * is 0, i.e. tokens*top_k <= 1024). */
size_t hm_permute_workspace_bytes(int64_t tokens, int32_t top_k, int64_t experts);
int hm_permute(const uint32_t* ids, const float* scores, int64_t tokens,
               int32_t top_k, int64_t experts, int32_t* counts,
               int32_t* offsets, int32_t* perm_tokens, float* perm_weights,
               int32_t* slots, void* workspace, void* stream);

/* ---- A4  Gather rows (src/core/runtime/MoERuntime.cpp:282-299) ----------
 * out[r,:] = in[rows[r],:]. */
int hm_gather_rows(const float* in, const int32_t* rows, int64_t count,
                   int64_t width, float* out, void* stream);

/* ---- A5/A5' op level (TensorBackend::matmulInt8Weights / matmul,
 * src/tensor/backend/CpuTensorBackend.cpp:87-190).  x [M x K] FP32,
 * q / w [K x N] row-major INPUT_OUTPUT, y [M x N].
 * hm_matmul_w8a32 uses the reference's W8A32 arithmetic,
 * acc += x * (float(q - zp) * scale) in FP32, with a bounded deterministic
 * split-K (hm_plan_int8_gemm); within 1e-5 + 1e-5|ref| of the CPU path. */
typedef struct hm_int8_gemm_plan {
    int32_t implementation; /* 1 = Reference (one lane per output),
                               2 = Cooperative (split-K partitions) */
    int64_t partitions;     /* bounded split-K: min(8, ceil(K/512)) */
    int64_t blocks;         /* workgroups launched */
    int64_t scratch_elements; /* FP32 split-K scratch, M*N*P if P > 1 */
} hm_int8_gemm_plan;
/* Launch plan, src/backend/cuda/Int8GemmPlan.cpp:29-53 (mode: 0 auto,
 * 1 reference, 2 cooperative). */
int hm_plan_int8_gemm(int64_t rows, int64_t inner, int64_t cols, int32_t mode,
                      hm_int8_gemm_plan* plan_out /* host */);
int hm_matmul_w8a32(const float* x, const int8_t* q, float scale, int32_t zp,
                    float* y, int64_t rows, int64_t inner, int64_t cols,
                    int32_t mode, float* scratch, size_t scratch_bytes,
                    void* stream);
int hm_matmul_f32(const float* x, const float* w, float* y, int64_t rows,
                  int64_t inner, int64_t cols, void* stream);

/* ---- A6  elementwise (Activation.cpp:44, CpuTensorBackend.cpp:192-220) */
int hm_silu(const float* x, float* y, int64_t n, void* stream);
int hm_mul(const float* a, const float* b, float* y, int64_t n, void* stream);
int hm_add(const float* a, const float* b, float* y, int64_t n, void* stream);

/* ---- A7  Combine (src/core/runtime/MoERuntime.cpp:308-325) --------------
 * out[t,:] = sum over the token's pairs in ascending expert id of
 * w * y_grouped[slot,:], float multiply then float add, starting from 0.
 * Bit-exact given y_grouped.  If residual != NULL, out = residual + sum
 * (TransformerBlock.cpp:101-104), the add done last. */
int hm_combine(const float* y_grouped, const uint32_t* ids,
               const int32_t* slots, const float* scores, int64_t tokens,
               int32_t top_k, int64_t width, const float* residual,
               float* out, void* stream);

/* ---- A8  INT8 packer (src/tensor/quantization/Quantization.cpp:45-79) on
 * the host: scale = max|w|/127 (1 if all zero), zp = 0,
 * q = int8(clamp(round(w/scale), -127, 127)).  Host pointers. */
int hm_quantize_int8_host(const float* w /* host */, int64_t n,
                          int8_t* q /* host */, float* scale /* host */,
                          int32_t* zero_point /* host */,
                          float* max_abs_error /* host, may be NULL */);

/* ---- A10  Device-resident expert table --------------------------------
 * The reference payload for expert e is gate [H x I] | up [H x I] |
 * down [I x H], row-major INPUT_OUTPUT (ExpertPacker.cpp:228-230,
 * WeightConverter.cpp:31-42).  hm_pack_layer re-lays it out once on the
 * device into the kernels' layout: each projection transposed to [N x K]
 * (K contiguous), experts back to back.  The packed table holds
 * 3*E*H*I elements of the same dtype. */
typedef struct hm_layer {
    int64_t experts, hidden, intermediate;
    int32_t dtype;              /* HM_DTYPE_INT8 or HM_DTYPE_FP32 */
    const void* packed;         /* output of hm_pack_layer */
    const float* scale;         /* [E x 3] {gate, up, down}, INT8 only */
    const int32_t* zero_point;  /* [E x 3], INT8 only */
} hm_layer;
size_t hm_packed_layer_bytes(int64_t experts, int64_t hidden,
                             int64_t intermediate, int32_t dtype);
int hm_pack_layer(const void* reference_payload, int64_t experts,
                  int64_t hidden, int64_t intermediate, int32_t dtype,
                  void* packed, void* stream);

/* ---- A5 block level + A11: the fused MoE block ------------------------
 * MoERuntime::executeBatch (src/core/runtime/MoERuntime.cpp:58-349) with all
 * experts device resident: route -> permute -> grouped SwiGLU experts ->
 * combine.  hidden [T x H] (post-RMSNorm), router_w [H x E].
 *
 * INT8 experts use the integer-limb arithmetic: activations are written as
 * per-row (gate/up) or per-128-column (down) fixed point split into
 * `limbs_x` / `limbs_z` balanced signed INT8 digits; every int32 partial is
 * exact; the FP32 result is within 1e-4 of the reference W8A32 path for
 * limbs >= 2 and bit-exact against the build's CPU restatement.
 * FP32 experts use FP32 arithmetic (within 1e-3 of the reference).
 *
 * Outputs (device, caller-owned; all but `out` may be NULL, in which case
 * the workspace copy is used):
 *   out [T x H]; ids, scores [T x k]; counts [E]; offsets [E+1];
 *   perm_tokens, perm_weights [T*k]; expert_out [T*k x H] (grouped order,
 *   the per-group expert outputs of BatchLayerExecutionResult);
 *   status: HM_STATUS_* bits (must be zeroed by the caller once; kernels
 *   only OR bits in).
 * The workspace must hold hm_moe_block_workspace_bytes(...) bytes. */
typedef struct hm_block_io {
    float* out;
    uint32_t* ids;
    float* scores;
    int32_t* counts;
    int32_t* offsets;
    int32_t* perm_tokens;
    float* perm_weights;
    float* expert_out;
    int32_t* status;
    const float* residual; /* optional: out = residual + MoE(hidden) */
    /* Optional profiling spans (the role of the reference's GpuEventQueue,
     * src/profiling/GpuEventQueue.hpp:17-69): HM_BLOCK_EVENTS hipEvent_t
     * handles recorded on `stream` at the stage boundaries
     * [start, routed, permuted, quantised, gate/up done, down done,
     * combined].  Events 3 and 4 bracket the gate/up kernels themselves:
     * they are taken at the first kernel's start and the last kernel's end
     * (hipExtLaunchKernelGGL), so their span is the stage's kernel time.
     * NULL = no recording. */
    void* const* events;
} hm_block_io;
#define HM_BLOCK_EVENTS 7
/* exec_flags: the HM_EXEC_* bits the calls will pass (the generic path needs
 * an extra [T*k x I] float buffer). */
size_t hm_moe_block_workspace_bytes(const hm_layer* layer, int64_t tokens,
                                    int32_t top_k, int32_t limbs_x,
                                    int32_t limbs_z, uint32_t exec_flags);
int hm_moe_block_forward(const hm_layer* layer, const float* hidden,
                         const float* router_w, int64_t tokens, int32_t top_k,
                         uint32_t route_flags, int32_t limbs_x,
                         int32_t limbs_z, const hm_block_io* io,
                         void* workspace, size_t workspace_bytes,
                         void* stream);

/* One MoE sub-layer of the transformer block
 * (src/transformer/runtime/TransformerBlock.cpp:88-104: RMSNorm.cpp:65-77
 * on the layer input, the MoE block on the normalised rows, the input added
 * back): io->out = h + MoE(RMSNorm(h; gamma, eps)).  normed [tokens x
 * hidden] receives RMSNorm(h) (hm_rmsnorm's values); it must not overlap h.
 * io->residual must be NULL or h.  Decode batches normalise inside the
 * router's first kernel (one launch fewer than hm_rmsnorm followed by
 * hm_moe_block_forward); other batches launch hm_rmsnorm first.  Same
 * workspace as hm_moe_block_forward. */
int hm_moe_layer_forward(const hm_layer* layer, const float* h,
                         const float* gamma, float eps, float* normed,
                         const float* router_w, int64_t tokens, int32_t top_k,
                         uint32_t route_flags, int32_t limbs_x,
                         int32_t limbs_z, const hm_block_io* io,
                         void* workspace, size_t workspace_bytes,
                         void* stream);

/* ---- The block without allocation ------------------------------------
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): hm_moe_block_forward with its workspace in a
 * library-owned device array of HM_NOALLOC_WORKSPACE_BYTES per GPU (held
 * from first use until the process ends).  Same arguments and results as
 * hm_moe_block_forward without the workspace; the caller still passes the
 * inputs and the outputs in `io`.  Returns HM_ERR_UNSUPPORTED, without
 * launching anything, when the call needs a larger workspace
 * (hm_moe_block_workspace_bytes > HM_NOALLOC_WORKSPACE_BYTES: decode
 * batches always fit, prefill batches up to a few hundred tokens at the
 * Qwen3-30B-A3B shape).  It allocates nothing and calls no allocating
 * routine.  All calls on one GPU share the array: calls that overlap on a
 * GPU (other streams, other host threads) race and must be serialised by
 * the caller. */
#define HM_NOALLOC_WORKSPACE_BYTES ((size_t)64 << 20)
int hm_moe_block_forward_noalloc(const hm_layer* layer, const float* hidden,
                                 const float* router_w, int64_t tokens,
                                 int32_t top_k, uint32_t route_flags,
                                 int32_t limbs_x, int32_t limbs_z,
                                 const hm_block_io* io, void* stream);

/* ---- Limb arithmetic at op level (build-owned, no reference counterpart):
 * quantise rows to digit planes and return exact int32 partials, so tests
 * can pin "INT8 int32 partials bit-exact" directly.
 * digits: [limbs x rows x inner] int8; scales [rows];
 * partials: [limbs x rows x cols] int32 of sum_k d * (q[k,c] - zp) with q in
 * the packed [cols x inner] (transposed) layout. */
int hm_limb_quantize_rows(const float* x, int64_t rows, int64_t inner,
                          int32_t limbs, int8_t* digits, float* scales,
                          void* stream);
int hm_limb_partials(const int8_t* digits, int64_t rows, int64_t inner,
                     int32_t limbs, const int8_t* q_packed, int32_t zp,
                     int64_t cols, int32_t* partials, void* stream);

/* ---- Test hooks --------------------------------------------------------
 * The device restatement of glibc expf used by the router softmax and SiLU,
 * evaluated elementwise (parity of the libm boundary). */
int hm_debug_expf(const float* x, float* y, int64_t n, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* HM_MOE_H */
