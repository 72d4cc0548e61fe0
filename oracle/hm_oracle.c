/*
 * hm_oracle.c -- CPU oracle for the MoE-block hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see hm_oracle.h).  Restates the reference CPU
 * path of SHOnnay/hypermoe-engine with the same loop orders and types.
 * Build: gcc -O3 -ffp-contract=off -fPIC -shared (no -march), like the
 * reference's default Release build, which emits no FMA on x86-64.
 *
 * The limb functions at the end restate this build's own INT8 arithmetic,
 * which has no reference counterpart.
 */
#include "hm_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define CHECK(cond, code) do { if (!(cond)) return (code); } while (0)

static int mul_ok(int64_t a, int64_t b) {
    return a >= 0 && b >= 0 && (a == 0 || b <= INT64_MAX / a);
}

/* transformer/norm/RMSNorm.cpp:65-77.  squareSum accumulates double(x)^2 in
 * ascending order; the float epsilon is promoted to double; the output is
 * float(double(x) * inverseRms * double(gamma)). */
int hmo_rmsnorm(const float* x, const float* gamma, float* y,
                int64_t rows, int64_t width, float eps) {
    CHECK(x && gamma && y && rows >= 0 && width > 0, HMO_E_INVALID);
    CHECK(isfinite(eps) && eps > 0.0F, HMO_E_INVALID); /* RMSNorm.cpp:22 */
    for (int64_t t = 0; t < rows; ++t) {
        const float* row = x + t * width;
        double square_sum = 0.0;
        for (int64_t i = 0; i < width; ++i) {
            const float v = row[i];
            square_sum += (double)v * v;
        }
        const double inverse_rms =
            1.0 / sqrt(square_sum / (double)width + (double)eps);
        for (int64_t i = 0; i < width; ++i) {
            y[t * width + i] = (float)(row[i] * inverse_rms * gamma[i]);
        }
    }
    return HMO_OK;
}

/* router/CpuRouterBackend.cpp:41-49 for one token. */
static int token_logits(const float* h, const float* w, int64_t hidden,
                        int64_t experts, float* scores) {
    for (int64_t e = 0; e < experts; ++e) {
        double score = 0.0;
        for (int64_t i = 0; i < hidden; ++i) {
            score += (double)h[i] * (double)w[i * experts + e];
        }
        if (!isfinite(score)) return HMO_E_RUNTIME; /* :47 */
        scores[e] = (float)score;
    }
    return HMO_OK;
}

int hmo_router_logits(const float* h, const float* w, int64_t tokens,
                      int64_t hidden, int64_t experts, float* logits) {
    CHECK(h && w && logits && tokens >= 0 && hidden > 0 && experts > 0,
          HMO_E_INVALID);
    for (int64_t t = 0; t < tokens; ++t) {
        const int rc = token_logits(h + t * hidden, w, hidden, experts,
                                    logits + t * experts);
        if (rc) return rc;
    }
    return HMO_OK;
}

/* Comparator of CpuRouterBackend.cpp:69-71: higher score first, equal scores
 * (including -0 == +0) by ascending expert id. */
static int ranks_before(const float* s, uint32_t a, uint32_t b) {
    return s[a] == s[b] ? a < b : s[a] > s[b];
}

/* router/CpuRouterBackend.cpp:35-91 for one token. */
static int route_token(const float* h, const float* w, int64_t hidden,
                       int64_t experts, int32_t top_k, int32_t softmax,
                       int32_t renorm, float* scores, uint8_t* taken,
                       uint32_t* ids, float* out_scores) {
    int rc = token_logits(h, w, hidden, experts, scores);
    if (rc) return rc;
    if (softmax) { /* :50-63 */
        float maximum = scores[0];
        for (int64_t e = 1; e < experts; ++e) {
            if (scores[e] > maximum) maximum = scores[e]; /* max_element */
        }
        double denominator = 0.0;
        for (int64_t e = 0; e < experts; ++e) {
            scores[e] = expf(scores[e] - maximum);
            denominator += scores[e];
        }
        if (!isfinite(denominator) || denominator <= 0.0) return HMO_E_RUNTIME;
        for (int64_t e = 0; e < experts; ++e) {
            scores[e] = (float)((double)scores[e] / denominator);
        }
    }
    /* partial_sort of the first k ids under ranks_before (:64-72).  The
     * comparator is a strict total order on distinct ids, so the selected
     * prefix is unique; repeated selection of the best remaining id yields
     * it in rank order. */
    memset(taken, 0, (size_t)experts);
    for (int32_t r = 0; r < top_k; ++r) {
        uint32_t best = UINT32_MAX;
        for (int64_t e = 0; e < experts; ++e) {
            if (taken[e]) continue;
            if (best == UINT32_MAX || ranks_before(scores, (uint32_t)e, best)) {
                best = (uint32_t)e;
            }
        }
        taken[best] = 1;
        ids[r] = best;
        out_scores[r] = scores[best];
    }
    if (renorm) { /* :80-89, std::accumulate(..., 0.0) in rank order */
        double sum = 0.0;
        for (int32_t r = 0; r < top_k; ++r) sum += out_scores[r];
        if (!isfinite(sum) || sum == 0.0) return HMO_E_RUNTIME;
        for (int32_t r = 0; r < top_k; ++r) {
            out_scores[r] = (float)((double)out_scores[r] / sum);
        }
    }
    return HMO_OK;
}

int hmo_route(const float* h, const float* w, int64_t tokens, int64_t hidden,
              int64_t experts, int32_t top_k, int32_t softmax, int32_t renorm,
              uint32_t* ids, float* scores) {
    /* RouterConfig::validate, router/RouterConfig.cpp:9-22 */
    CHECK(experts > 0 && experts <= (int64_t)UINT32_MAX, HMO_E_INVALID);
    CHECK(top_k > 0 && top_k <= experts, HMO_E_INVALID);
    CHECK(h && w && ids && scores && tokens >= 0 && hidden > 0, HMO_E_INVALID);
    float* work = (float*)malloc((size_t)experts * sizeof(float));
    uint8_t* taken = (uint8_t*)malloc((size_t)experts);
    if (!work || !taken) { free(work); free(taken); return HMO_E_RUNTIME; }
    int rc = HMO_OK;
    for (int64_t t = 0; t < tokens && rc == HMO_OK; ++t) {
        rc = route_token(h + t * hidden, w, hidden, experts, top_k, softmax,
                         renorm, work, taken, ids + t * top_k,
                         scores + t * top_k);
    }
    free(work);
    free(taken);
    return rc;
}

/* router/CpuRouterBackend.cpp:140-159.  Appending (t, score) to group
 * ids[t, r] while walking tokens ascending and then sorting groups by expert
 * id is a stable counting sort by expert id over the token-major pairs. */
int hmo_group(const uint32_t* ids, const float* scores, int64_t tokens,
              int32_t top_k, int64_t experts, int32_t* counts, int32_t* offsets,
              int32_t* perm_tokens, float* perm_weights, int32_t* slots) {
    CHECK(ids && scores && counts && offsets && perm_tokens && perm_weights,
          HMO_E_INVALID);
    CHECK(tokens >= 0 && top_k > 0 && experts > 0 && mul_ok(tokens, top_k),
          HMO_E_INVALID);
    CHECK(tokens * top_k <= INT32_MAX, HMO_E_OVERFLOW);
    memset(counts, 0, (size_t)experts * sizeof(int32_t));
    for (int64_t p = 0; p < tokens * top_k; ++p) {
        CHECK(ids[p] < (uint64_t)experts, HMO_E_INVALID);
        counts[ids[p]]++;
    }
    offsets[0] = 0;
    for (int64_t e = 0; e < experts; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int32_t* fill = (int32_t*)malloc((size_t)experts * sizeof(int32_t));
    if (!fill) return HMO_E_RUNTIME;
    memcpy(fill, offsets, (size_t)experts * sizeof(int32_t));
    for (int64_t t = 0; t < tokens; ++t) {
        for (int32_t r = 0; r < top_k; ++r) {
            const int64_t p = t * top_k + r;
            const int32_t pos = fill[ids[p]]++;
            perm_tokens[pos] = (int32_t)t;
            perm_weights[pos] = scores[p];
            if (slots) slots[p] = pos;
        }
    }
    free(fill);
    return HMO_OK;
}

/* tensor/backend/CpuTensorBackend.cpp:120-129 */
void hmo_matmul_f32(const float* x, const float* w, float* y,
                    int64_t rows, int64_t inner, int64_t cols) {
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t c = 0; c < cols; ++c) {
            float sum = 0.0F;
            for (int64_t k = 0; k < inner; ++k) {
                sum += x[r * inner + k] * w[k * cols + c];
            }
            y[r * cols + c] = sum;
        }
    }
}

/* quantization::validateParameters for INT8, Quantization.cpp:24-35 */
static int valid_qparams(float scale, int32_t zp) {
    return isfinite(scale) && scale > 0.0F && zp >= -128 && zp <= 127;
}

/* tensor/backend/CpuTensorBackend.cpp:173-186 */
int hmo_matmul_w8a32(const float* x, const int8_t* q, float scale, int32_t zp,
                     float* y, int64_t rows, int64_t inner, int64_t cols) {
    CHECK(valid_qparams(scale, zp), HMO_E_INVALID);
    CHECK(x && q && y, HMO_E_INVALID);
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t c = 0; c < cols; ++c) {
            float sum = 0.0F;
            for (int64_t k = 0; k < inner; ++k) {
                const int32_t quantized = (int32_t)q[k * cols + c];
                const float weight = (float)(quantized - zp) * scale;
                sum += x[r * inner + k] * weight;
            }
            y[r * cols + c] = sum;
        }
    }
    return HMO_OK;
}

/* tensor/activation/Activation.cpp:44 */
static float silu1(float v) { return v / (1.0F + expf(-v)); }

void hmo_silu(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = silu1(x[i]);
}

void hmo_mul(const float* a, const float* b, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = a[i] * b[i];
}

void hmo_add(const float* a, const float* b, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = a[i] + b[i];
}

/* tensor/quantization/Quantization.cpp:45-79 */
int hmo_quantize_int8(const float* w, int64_t n, int8_t* q, float* scale,
                      int32_t* zero_point, float* max_abs_error) {
    CHECK(w && q && scale && zero_point && n > 0, HMO_E_INVALID);
    float maximum = 0.0F;
    for (int64_t i = 0; i < n; ++i) {
        CHECK(isfinite(w[i]), HMO_E_INVALID);
        const float magnitude = fabsf(w[i]);
        if (magnitude > maximum) maximum = magnitude; /* std::max */
    }
    const float s = maximum == 0.0F ? 1.0F : maximum / 127.0F;
    float max_error = 0.0F;
    for (int64_t i = 0; i < n; ++i) {
        float rounded = roundf(w[i] / s); /* std::round: half away from 0 */
        if (rounded < -127.0F) rounded = -127.0F;
        if (rounded > 127.0F) rounded = 127.0F;
        q[i] = (int8_t)rounded;
        const float reconstructed = (float)((int32_t)q[i] - 0) * s;
        const float error = fabsf(w[i] - reconstructed);
        if (error > max_error) max_error = error;
    }
    *scale = s;
    *zero_point = 0;
    if (max_abs_error) *max_abs_error = max_error;
    return HMO_OK;
}

static int layer_ok(const hmo_layer* L) {
    if (!L || !L->payload || L->experts <= 0 || L->hidden <= 0 ||
        L->intermediate <= 0) return 0;
    if (L->is_int8) {
        if (!L->scale || !L->zero_point) return 0;
        for (int64_t i = 0; i < L->experts * 3; ++i) {
            if (!valid_qparams(L->scale[i], L->zero_point[i])) return 0;
        }
    }
    return 1;
}

/* experts/ExpertExecutor.cpp:97-131: gate, up, silu(gate), act*up, down. */
int hmo_expert_mlp(const hmo_layer* layer, int64_t expert, const float* x,
                   int64_t rows, float* y) {
    CHECK(layer_ok(layer) && expert >= 0 && expert < layer->experts && x && y,
          HMO_E_INVALID);
    const int64_t H = layer->hidden, I = layer->intermediate;
    const size_t inter = (size_t)(rows * I);
    float* gate = (float*)malloc(inter * sizeof(float));
    float* up = (float*)malloc(inter * sizeof(float));
    float* act = (float*)malloc(inter * sizeof(float));
    float* gated = (float*)malloc(inter * sizeof(float));
    int rc = HMO_OK;
    if (!gate || !up || !act || !gated) { rc = HMO_E_RUNTIME; goto done; }
    if (layer->is_int8) {
        const int8_t* base = (const int8_t*)layer->payload + expert * 3 * H * I;
        const float* s = layer->scale + expert * 3;
        const int32_t* z = layer->zero_point + expert * 3;
        rc = hmo_matmul_w8a32(x, base, s[0], z[0], gate, rows, H, I);
        if (!rc) rc = hmo_matmul_w8a32(x, base + H * I, s[1], z[1], up, rows, H, I);
        if (rc) goto done;
        hmo_silu(gate, act, rows * I);
        hmo_mul(act, up, gated, rows * I);
        rc = hmo_matmul_w8a32(gated, base + 2 * H * I, s[2], z[2], y, rows, I, H);
    } else {
        const float* base = (const float*)layer->payload + expert * 3 * H * I;
        hmo_matmul_f32(x, base, gate, rows, H, I);
        hmo_matmul_f32(x, base + H * I, up, rows, H, I);
        hmo_silu(gate, act, rows * I);
        hmo_mul(act, up, gated, rows * I);
        hmo_matmul_f32(gated, base + 2 * H * I, y, rows, I, H);
    }
done:
    free(gate); free(up); free(act); free(gated);
    return rc;
}

/* core/runtime/MoERuntime.cpp:312-324 */
int hmo_combine(const float* y_grouped, const int32_t* offsets,
                const int32_t* perm_tokens, const float* perm_weights,
                int64_t experts, int64_t tokens, int64_t width, float* out) {
    CHECK(y_grouped && offsets && perm_tokens && perm_weights && out,
          HMO_E_INVALID);
    memset(out, 0, (size_t)(tokens * width) * sizeof(float));
    for (int64_t e = 0; e < experts; ++e) {
        for (int32_t row = offsets[e]; row < offsets[e + 1]; ++row) {
            const int64_t t = perm_tokens[row];
            const float w = perm_weights[row];
            CHECK(t >= 0 && t < tokens, HMO_E_INVALID);
            for (int64_t i = 0; i < width; ++i) {
                out[t * width + i] += w * y_grouped[(int64_t)row * width + i];
            }
        }
    }
    return HMO_OK;
}

typedef int (*mlp_fn)(const hmo_layer*, int64_t, const float*, int64_t,
                      float*, int32_t, int32_t);

static int ref_mlp(const hmo_layer* l, int64_t e, const float* x, int64_t rows,
                   float* y, int32_t a, int32_t b) {
    (void)a; (void)b;
    return hmo_expert_mlp(l, e, x, rows, y);
}

static int limb_mlp(const hmo_layer* l, int64_t e, const float* x,
                    int64_t rows, float* y, int32_t a, int32_t b) {
    return hmo_limb_expert_mlp(l, e, x, rows, a, b, y);
}

/* core/runtime/MoERuntime.cpp:58-349 with the residency machinery
 * (scheduler, leases) removed: every expert is resident. */
static int moe_block(const hmo_layer* layer, const float* hidden,
                     const float* router_w, int64_t tokens, int32_t top_k,
                     int32_t softmax, int32_t renorm, float* out,
                     uint32_t* ids_out, float* scores_out, mlp_fn mlp,
                     int32_t la, int32_t lb) {
    CHECK(layer_ok(layer) && hidden && router_w && out, HMO_E_INVALID);
    CHECK(tokens > 0, HMO_E_INVALID); /* BatchRouterDecision::valid */
    const int64_t H = layer->hidden, E = layer->experts;
    const int64_t pairs = tokens * top_k;
    uint32_t* ids = (uint32_t*)malloc((size_t)pairs * sizeof(uint32_t));
    float* scores = (float*)malloc((size_t)pairs * sizeof(float));
    int32_t* counts = (int32_t*)malloc((size_t)E * sizeof(int32_t));
    int32_t* offsets = (int32_t*)malloc((size_t)(E + 1) * sizeof(int32_t));
    int32_t* ptok = (int32_t*)malloc((size_t)pairs * sizeof(int32_t));
    float* pw = (float*)malloc((size_t)pairs * sizeof(float));
    float* xg = (float*)malloc((size_t)(tokens * H) * sizeof(float));
    float* yg = (float*)malloc((size_t)(pairs * H) * sizeof(float));
    int rc = HMO_OK;
    if (!ids || !scores || !counts || !offsets || !ptok || !pw || !xg || !yg) {
        rc = HMO_E_RUNTIME;
        goto done;
    }
    rc = hmo_route(hidden, router_w, tokens, H, E, top_k, softmax, renorm, ids,
                   scores);
    if (rc) goto done;
    rc = hmo_group(ids, scores, tokens, top_k, E, counts, offsets, ptok, pw,
                   NULL);
    if (rc) goto done;
    for (int64_t e = 0; e < E && rc == HMO_OK; ++e) {
        const int64_t n = counts[e];
        if (n == 0) continue;
        for (int64_t r = 0; r < n; ++r) { /* gather, MoERuntime.cpp:288-298 */
            memcpy(xg + r * H, hidden + (int64_t)ptok[offsets[e] + r] * H,
                   (size_t)H * sizeof(float));
        }
        rc = mlp(layer, e, xg, n, yg + (int64_t)offsets[e] * H, la, lb);
    }
    if (rc) goto done;
    rc = hmo_combine(yg, offsets, ptok, pw, E, tokens, H, out);
    if (ids_out) memcpy(ids_out, ids, (size_t)pairs * sizeof(uint32_t));
    if (scores_out) memcpy(scores_out, scores, (size_t)pairs * sizeof(float));
done:
    free(ids); free(scores); free(counts); free(offsets);
    free(ptok); free(pw); free(xg); free(yg);
    return rc;
}

int hmo_moe_block(const hmo_layer* layer, const float* hidden,
                  const float* router_w, int64_t tokens, int32_t top_k,
                  int32_t softmax, int32_t renorm, float* out,
                  uint32_t* ids, float* scores) {
    return moe_block(layer, hidden, router_w, tokens, top_k, softmax, renorm,
                     out, ids, scores, ref_mlp, 0, 0);
}

/* ---------------------------------------------------------------------- */
/* Build-owned integer-limb arithmetic (no reference counterpart).         */
/* ---------------------------------------------------------------------- */

static int32_t limb_range(int32_t limbs) {
    /* 127 * (256^L - 1) / 255: the largest |n| whose balanced base-256
     * digits all fit [-128, 127] symmetrically. */
    return limbs == 1 ? 127 : limbs == 2 ? 32639 : 8355711;
}

int hmo_limb_quantize(const float* x, int64_t rows, int64_t n, int64_t ld,
                      int32_t limbs, int8_t* digits, float* scales) {
    CHECK(x && digits && scales && rows >= 0 && n > 0 && ld >= n, HMO_E_INVALID);
    CHECK(limbs >= 1 && limbs <= 3, HMO_E_INVALID);
    const int32_t range = limb_range(limbs);
    const float frange = (float)range;
    for (int64_t r = 0; r < rows; ++r) {
        const float* row = x + r * ld;
        float amax = 0.0F;
        for (int64_t k = 0; k < n; ++k) amax = fmaxf(amax, fabsf(row[k]));
        const float inv = amax > 0.0F ? frange / amax : 0.0F;
        scales[r] = amax > 0.0F ? amax / frange : 0.0F;
        for (int64_t k = 0; k < n; ++k) {
            float v = rintf(row[k] * inv);
            v = fminf(fmaxf(v, -frange), frange);
            int32_t value = (int32_t)v;
            for (int32_t l = 0; l < limbs; ++l) {
                const int32_t d = ((value + 128) & 255) - 128;
                digits[((int64_t)l * rows + r) * n + k] = (int8_t)d;
                value = (value - d) / 256;
            }
        }
    }
    return HMO_OK;
}

int hmo_limb_partials(const int8_t* digits, int64_t rows, int64_t inner,
                      int32_t limbs, const int8_t* q, int32_t zp, int64_t cols,
                      int32_t* partials) {
    CHECK(digits && q && partials && limbs >= 1 && limbs <= 3, HMO_E_INVALID);
    for (int32_t l = 0; l < limbs; ++l) {
        for (int64_t r = 0; r < rows; ++r) {
            const int8_t* d = digits + ((int64_t)l * rows + r) * inner;
            for (int64_t c = 0; c < cols; ++c) {
                int64_t acc = 0;
                for (int64_t k = 0; k < inner; ++k) {
                    acc += (int64_t)d[k] * ((int64_t)q[k * cols + c] - zp);
                }
                CHECK(acc >= INT32_MIN && acc <= INT32_MAX, HMO_E_OVERFLOW);
                partials[((int64_t)l * rows + r) * cols + c] = (int32_t)acc;
            }
        }
    }
    return HMO_OK;
}

/* c = (float)P_{L-1}; c = fmaf(c, 256, (float)P_l) for l = L-2 .. 0 */
static float recombine(const int32_t* p, int64_t plane, int32_t limbs) {
    float c = (float)p[(int64_t)(limbs - 1) * plane];
    for (int32_t l = limbs - 2; l >= 0; --l) {
        c = fmaf(c, 256.0F, (float)p[(int64_t)l * plane]);
    }
    return c;
}

int hmo_limb_matmul(const float* x, int64_t rows, int64_t inner,
                    const int8_t* q, float scale, int32_t zp, int64_t cols,
                    int32_t limbs, float* y) {
    CHECK(valid_qparams(scale, zp), HMO_E_INVALID);
    CHECK(x && q && y && rows >= 0 && inner > 0 && cols > 0, HMO_E_INVALID);
    if (rows == 0) return HMO_OK;
    int8_t* dg = (int8_t*)malloc((size_t)(limbs * rows * inner));
    float* s = (float*)malloc((size_t)rows * sizeof(float));
    int32_t* p = (int32_t*)malloc((size_t)(limbs * rows * cols) * sizeof(int32_t));
    int rc = (dg && s && p) ? HMO_OK : HMO_E_RUNTIME;
    if (!rc) rc = hmo_limb_quantize(x, rows, inner, inner, limbs, dg, s);
    if (!rc) rc = hmo_limb_partials(dg, rows, inner, limbs, q, zp, cols, p);
    if (!rc) {
        for (int64_t r = 0; r < rows; ++r) {
            const float alpha = s[r] * scale;
            for (int64_t c = 0; c < cols; ++c) {
                y[r * cols + c] = recombine(p + r * cols + c, rows * cols, limbs) * alpha;
            }
        }
    }
    free(dg); free(s); free(p);
    return rc;
}

int hmo_limb_expert_mlp(const hmo_layer* layer, int64_t expert, const float* x,
                        int64_t rows, int32_t limbs_x, int32_t limbs_z,
                        float* y) {
    CHECK(layer_ok(layer) && layer->is_int8 && expert >= 0 &&
          expert < layer->experts && x && y, HMO_E_INVALID);
    CHECK(limbs_x >= 1 && limbs_x <= 3 && limbs_z >= 1 && limbs_z <= 3,
          HMO_E_INVALID);
    const int64_t H = layer->hidden, I = layer->intermediate;
    const int8_t* base = (const int8_t*)layer->payload + expert * 3 * H * I;
    const float* sc = layer->scale + expert * 3;
    const int32_t* zp = layer->zero_point + expert * 3;
    const size_t inter = (size_t)(rows * I);
    float* g = (float*)malloc(inter * sizeof(float));
    float* u = (float*)malloc(inter * sizeof(float));
    float* z = (float*)malloc(inter * sizeof(float));
    int rc = (g && u && z) ? HMO_OK : HMO_E_RUNTIME;
    if (!rc) rc = hmo_limb_matmul(x, rows, H, base, sc[0], zp[0], I, limbs_x, g);
    if (!rc) rc = hmo_limb_matmul(x, rows, H, base + H * I, sc[1], zp[1], I, limbs_x, u);
    if (!rc) {
        for (size_t i = 0; i < inter; ++i) z[i] = silu1(g[i]) * u[i];
        rc = hmo_limb_matmul(z, rows, I, base + 2 * H * I, sc[2], zp[2], H, limbs_z, y);
    }
    free(g); free(u); free(z);
    return rc;
}

int hmo_moe_block_limbs(const hmo_layer* layer, const float* hidden,
                        const float* router_w, int64_t tokens, int32_t top_k,
                        int32_t softmax, int32_t renorm, int32_t limbs_x,
                        int32_t limbs_z, float* out, uint32_t* ids,
                        float* scores) {
    CHECK(layer && layer->is_int8, HMO_E_INVALID);
    return moe_block(layer, hidden, router_w, tokens, top_k, softmax, renorm,
                     out, ids, scores, limb_mlp, limbs_x, limbs_z);
}
