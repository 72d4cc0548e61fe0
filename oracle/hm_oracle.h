/*
 * hm_oracle.h -- CPU oracle for the MoE-block hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product links, loads or calls
 * this library.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may use it, and only as the checker or the timed CPU
 * baseline.
 *
 * Two kinds of functions live here:
 *
 *   1. A restatement of the reference CPU path (SHOnnay/hypermoe-engine),
 *      same loop orders and the same float/double types, compiled with
 *      -O3 -ffp-contract=off and no -march (the reference's default Release
 *      flags emit no FMA on x86-64).  Each function cites the reference
 *      file:line it follows.  Pinned bit-for-bit against golden vectors
 *      written by the compiled reference (tests/golden, oracle/_ref).
 *
 *   2. A restatement of the build's own integer-limb arithmetic for the INT8
 *      expert GEMMs (hmo_limb_*).  The reference has no counterpart: it
 *      computes W8A32 in FP32.  These are pinned by brute-force int64 dot
 *      products on small inputs and by tolerance against (1).
 *
 * All functions return 0 on success or a negative HMO_E_* code, mirroring
 * the reference's exception categories.
 */
#ifndef HM_ORACLE_H
#define HM_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    HMO_OK = 0,
    HMO_E_INVALID = -1,  /* std::invalid_argument */
    HMO_E_OVERFLOW = -2, /* std::overflow_error   */
    HMO_E_RUNTIME = -3   /* std::runtime_error (non-finite router score, ...) */
};

/* RMSNorm CPU branch, transformer/norm/RMSNorm.cpp:65-77. */
int hmo_rmsnorm(const float* x, const float* gamma, float* y,
                int64_t rows, int64_t width, float eps);

/* Router logits, router/CpuRouterBackend.cpp:41-49: double accumulation in
 * ascending feature order, rounded to float.  logits is [T x E]. */
int hmo_router_logits(const float* h, const float* w, int64_t tokens,
                      int64_t hidden, int64_t experts, float* logits);

/* Full per-token routing, router/CpuRouterBackend.cpp:35-91.
 * ids/scores are [T x k], in rank order.  softmax: 1 = Softmax, 0 = None. */
int hmo_route(const float* h, const float* w, int64_t tokens, int64_t hidden,
              int64_t experts, int32_t top_k, int32_t softmax, int32_t renorm,
              uint32_t* ids, float* scores);

/* Grouping, router/CpuRouterBackend.cpp:140-159: groups sorted by expert id,
 * tokens ascending inside a group.  counts[E], offsets[E+1] (exclusive
 * prefix), perm_tokens / perm_weights [T*k] in group order.  slots [T*k]
 * (optional) receives, for pair (t, r), its row in the grouped order. */
int hmo_group(const uint32_t* ids, const float* scores, int64_t tokens,
              int32_t top_k, int64_t experts, int32_t* counts, int32_t* offsets,
              int32_t* perm_tokens, float* perm_weights, int32_t* slots);

/* FP32 GEMM, tensor/backend/CpuTensorBackend.cpp:120-129. */
void hmo_matmul_f32(const float* x, const float* w, float* y,
                    int64_t rows, int64_t inner, int64_t cols);

/* W8A32 GEMM, tensor/backend/CpuTensorBackend.cpp:173-186. */
int hmo_matmul_w8a32(const float* x, const int8_t* q, float scale, int32_t zp,
                     float* y, int64_t rows, int64_t inner, int64_t cols);

/* SiLU, tensor/activation/Activation.cpp:44; mul/add,
 * tensor/backend/CpuTensorBackend.cpp:202-204, 217-219. */
void hmo_silu(const float* x, float* y, int64_t n);
void hmo_mul(const float* a, const float* b, float* y, int64_t n);
void hmo_add(const float* a, const float* b, float* y, int64_t n);

/* INT8 packer, tensor/quantization/Quantization.cpp:45-79. */
int hmo_quantize_int8(const float* w, int64_t n, int8_t* q, float* scale,
                      int32_t* zero_point, float* max_abs_error);

/* Expert weights for one layer.  Expert e occupies one contiguous payload:
 * gate [H x I] | up [H x I] | down [I x H], each row-major INPUT_OUTPUT
 * (tools/model_convert/ExpertPacker.cpp:228-230, WeightConverter.cpp:31-42).
 * For INT8 payloads scale/zp hold {gate, up, down} per expert: [E x 3]. */
typedef struct {
    int64_t experts, hidden, intermediate;
    int32_t is_int8;
    const void* payload;      /* int8_t or float, E * 3*H*I elements */
    const float* scale;       /* [E x 3] (INT8 only) */
    const int32_t* zero_point;/* [E x 3] (INT8 only) */
} hmo_layer;

/* ExpertMlpExecutor::execute, experts/ExpertExecutor.cpp:97-131, for one
 * expert on `rows` gathered input rows. */
int hmo_expert_mlp(const hmo_layer* layer, int64_t expert, const float* x,
                   int64_t rows, float* y);

/* MoERuntime::executeBatch CPU path, core/runtime/MoERuntime.cpp:58-349:
 * route, group, gather, expert MLP per group in ascending expert id, combine
 * (:312-324).  out [T x H]; ids/scores [T x k] (optional). */
int hmo_moe_block(const hmo_layer* layer, const float* hidden,
                  const float* router_w, int64_t tokens, int32_t top_k,
                  int32_t softmax, int32_t renorm, float* out,
                  uint32_t* ids, float* scores);

/* Combine, core/runtime/MoERuntime.cpp:312-324, over grouped expert outputs
 * y_grouped [T*k x H] in group order: out is zeroed, then groups are
 * accumulated in ascending expert order with separate float mul and add. */
int hmo_combine(const float* y_grouped, const int32_t* offsets,
                const int32_t* perm_tokens, const float* perm_weights,
                int64_t experts, int64_t tokens, int64_t width, float* out);

/* ------------------------------------------------------------------------
 * Build-owned integer-limb INT8 arithmetic (no reference counterpart).
 *
 * An FP32 row segment x[0..n) is written as fixed point n_k*s with
 * |n_k| <= N(L) = 127*(256^L-1)/255 and split into L balanced signed digits
 * n_k = sum_l d_{l,k} 256^l, d in [-128,127]:
 *   amax = max|x_k| (float); amax == 0 => all digits 0, s = 0
 *   inv  = (float)N(L) / amax            (float division)
 *   n_k  = clamp(rintf(x_k * inv), -N, N) (float multiply, ties-to-even)
 *   s    = amax / (float)N(L)            (float division)
 * Int32 partials of one limb against INT8 weights with zero point zp:
 *   P_l[n] = sum_k d_{l,k} * (q[k,n] - zp)      (exact)
 * Recombination (float, explicit fmaf, fixed order):
 *   c = (float)P_{L-1}; for l = L-2..0: c = fmaf(c, 256, (float)P_l)
 *   alpha = s * scale_w;  value = c * alpha
 * Both GEMMs use one segment per row: the gate/up GEMM quantises each
 * token row of X (whole H), the down GEMM each row of Z = silu(G)*U (whole
 * I), so every partial is one exact integer per (row, column) and the
 * recombination above gives the output directly.
 * ---------------------------------------------------------------------- */

/* Quantise `rows` segments of length n (row stride ld) to L digit planes:
 * digits[(l*rows + r)*n + k]; scales[r] = s. */
int hmo_limb_quantize(const float* x, int64_t rows, int64_t n, int64_t ld,
                      int32_t limbs, int8_t* digits, float* scales);

/* Exact limb partials by brute-force int64 dot products (checked to fit
 * int32): partials[(l*rows + r)*cols + c]. q is [inner x cols] row-major. */
int hmo_limb_partials(const int8_t* digits, int64_t rows, int64_t inner,
                      int32_t limbs, const int8_t* q, int32_t zp, int64_t cols,
                      int32_t* partials);

/* Limb W8A32 replacement for one projection with one segment per row:
 * y[r,c] = recombine(P)[r,c] * (s_r * scale). */
int hmo_limb_matmul(const float* x, int64_t rows, int64_t inner,
                    const int8_t* q, float scale, int32_t zp, int64_t cols,
                    int32_t limbs, float* y);

/* Expert MLP in limb arithmetic: G and U with limbs_x digits per X row,
 * Z = SiLU(G)*U in float (Activation.cpp:44 then CpuTensorBackend::mul),
 * down with limbs_z digits per Z row. */
int hmo_limb_expert_mlp(const hmo_layer* layer, int64_t expert, const float* x,
                        int64_t rows, int32_t limbs_x, int32_t limbs_z,
                        float* y);

/* The MoE block with the limb expert MLP in place of the W8A32 one; routing,
 * grouping and combine are the reference's. */
int hmo_moe_block_limbs(const hmo_layer* layer, const float* hidden,
                        const float* router_w, int64_t tokens, int32_t top_k,
                        int32_t softmax, int32_t renorm, int32_t limbs_x,
                        int32_t limbs_z, float* out, uint32_t* ids,
                        float* scores);

#ifdef __cplusplus
}
#endif
#endif /* HM_ORACLE_H */
