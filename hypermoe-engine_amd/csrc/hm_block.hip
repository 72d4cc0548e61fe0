// hm_block.hip -- the fused MoE block entry (MoERuntime::executeBatch,
// src/core/runtime/MoERuntime.cpp:58-349, with every expert device
// resident) and the host-side INT8 packer.
#include "hm_device.h"

#include <limits.h>
#include <math.h>

#include <cmath>


int hm_launch_rmsnorm(const float* x, const float* gamma, float* y, int64_t rows,
                      int64_t width, float eps, bool force_seq, void* stream);
int hm_launch_quantize_rows(const float* x, int64_t rows, int64_t n, int32_t limbs,
                            int8_t* digits, float* scales, int32_t* dsum,
                            hipStream_t stream);

int hm_launch_gateup_i8(const hm_layer* layer, int32_t lx, int32_t lz, const int8_t* xdig,
                        const float* xscale, const int32_t* xdsum, int64_t tokens,
                        const int32_t* counts, const int32_t* offsets,
                        const int32_t* perm_tokens, int64_t R, int8_t* zdig, float* zscale,
                        int32_t* zdsum, float* gu, bool force_generic, bool split_k,
                        hipStream_t stream);
int hm_launch_down_i8(const hm_layer* layer, int32_t lx, int32_t lz, const int32_t* counts,
                      const int32_t* offsets, int64_t R, const int8_t* zdig,
                      const float* zscale, const int32_t* zdsum, float* y,
                      bool force_generic, bool split_k, hipStream_t stream);
int hm_launch_gateup_f32(const hm_layer* layer, const float* hidden, const int32_t* counts,
                         const int32_t* offsets, const int32_t* perm_tokens, int64_t R,
                         float* zf, hipStream_t stream);
int hm_launch_down_f32(const hm_layer* layer, const int32_t* counts, const int32_t* offsets,
                       int64_t R, const float* zf, float* y, hipStream_t stream);
bool hm_gemv_shape_ok(int64_t H, int64_t I);
int hm_launch_gateup_gemv(const hm_layer* L, const float* hidden, const int32_t* counts,
                          const int32_t* offsets, const int32_t* perm_tokens, int64_t tokens,
                          int64_t pairs, float* z, hipStream_t s);
int hm_launch_down_gemv(const hm_layer* L, const float* z, const int32_t* counts,
                        const int32_t* offsets, int64_t pairs, float* y, hipStream_t s);
bool hm_gemv_combine_ok(int64_t tokens, int32_t top_k, int64_t H, int64_t I);
bool hm_gemv_f32_ok(const hm_layer* L, const void* x);
int hm_launch_gateup_gemv_f32(const hm_layer* L, const float* hidden, const int32_t* counts,
                              const int32_t* offsets, const int32_t* perm_tokens,
                              int64_t pairs, float* z, hipStream_t s);
int hm_launch_down_gemv_f32(const hm_layer* L, const float* z, const int32_t* counts,
                            const int32_t* offsets, int64_t pairs, float* y, hipStream_t s);
int hm_launch_down_combine_gemv(const hm_layer* L, const float* z, const int32_t* counts,
                                const uint32_t* ids, const int32_t* slots, const float* scores,
                                const float* residual, int64_t tokens, int32_t top_k,
                                float* y_out, float* out, hipStream_t s);
extern "C" __attribute__((visibility("hidden"))) int hm_router_topk_quant(const float* h, const float* w, int64_t tokens, int64_t hidden,
                         int64_t experts, int32_t top_k, uint32_t flags, uint32_t* ids,
                         float* scores, float* logits_out, int32_t* status, void* route_ws,
                         const hm_row_quant* xq, bool* quantized, int32_t* hist,
                         bool* counted, void* stream);
extern "C" __attribute__((visibility("hidden"))) int hm_permute_counted(const uint32_t* ids, const float* scores, int64_t tokens,
                       int32_t top_k, int64_t experts, int32_t* counts, int32_t* offsets,
                       int32_t* perm_tokens, float* perm_weights, int32_t* slots,
                       void* workspace, bool counted, void* stream);
bool hm_select_gateup_ok(const hm_layer* L, int32_t top_k);
int hm_route_partials_decode(const float* h, const float* w, int64_t hidden, int64_t experts,
                             int32_t top_k, uint32_t flags, int32_t* status, void* route_ws,
                             const hm_decode_fusion* fused, const hm_norm_fold* norm,
                             void* stream);
int hm_launch_select_gateup(const float* x, const float* w, int32_t top_k, uint32_t flags,
                            uint32_t* ids, float* scores, int32_t* status, void* route_ws,
                            int32_t* counts, int32_t* offsets, int32_t* perm_tokens,
                            float* perm_weights, int32_t* slots, const hm_layer* L, float* z,
                            hipStream_t stream);
int hm_route_permute_decode(const float* h, const float* w, int64_t tokens, int64_t hidden,
                            int64_t experts, int32_t top_k, uint32_t flags, uint32_t* ids,
                            float* scores, int32_t* status, void* route_ws,
                            const hm_decode_fusion* fused, const hm_norm_fold* norm,
                            const hm_row_quant* xq, bool* quantized, void* stream);

namespace {

constexpr size_t kAlign = 256;

// Clears the workspace status word (a kernel, not a memset node, so the
// sequence stays safe to capture in a HIP graph).
__global__ void zero_status_kernel(int32_t* status) { *status = 0; }

size_t align_up(size_t v) { return (v + kAlign - 1) & ~(kAlign - 1); }

// Sequential carve of the workspace; every region 256-byte aligned.
struct Carve {
    char* base;
    size_t used = 0;
    explicit Carve(void* b) : base(static_cast<char*>(b)) {}
    template <typename T>
    T* take(size_t count) {
        T* p = base ? reinterpret_cast<T*>(base + used) : nullptr;
        used += align_up(count * sizeof(T));
        return p;
    }
};

struct BlockPlan {
    void* route_ws;
    void* permute_ws;
    uint32_t* ids;
    float* scores;
    int32_t* counts;
    int32_t* offsets;
    int32_t* perm_tokens;
    float* perm_weights;
    int32_t* slots;
    int8_t* xdig;
    float* xscale;
    int32_t* xdsum;
    int8_t* zdig;
    float* zscale;
    int32_t* zdsum;
    float* zf;
    float* gu;  // INT8 limb path: gate | up values [P x 2I], aliasing y
    float* y;
    int32_t* status;
    int32_t* counters;  // decode: the fused select's completion counter
};

// Decode-size INT8 blocks of at most HM_GEMV_MAX_PAIRS (token, expert) pairs
// take the W8A32 GEMV kernels; larger decode blocks the limb GEMMs (their
// weight streams run faster through the ring kernels' LDS stages once most
// experts see a row or two: C3-16 gate/up 54.5 against 60.5 us).
bool use_gemv(const hm_layer* L, int64_t T, int32_t k, uint32_t flags) {
    return L->dtype == HM_DTYPE_INT8 && (flags & (HM_EXEC_GENERIC | HM_EXEC_LIMBS)) == 0 &&
           T <= HM_GEMV_MAX_TOKENS && T * k <= HM_GEMV_MAX_PAIRS &&
           hm_gemv_shape_ok(L->hidden, L->intermediate);
}

bool layer_valid(const hm_layer* L) {
    if (!L || !L->packed || L->experts <= 0 || L->hidden <= 0 || L->intermediate <= 0)
        return false;
    if (L->dtype == HM_DTYPE_INT8) return L->scale && L->zero_point;
    return L->dtype == HM_DTYPE_FP32;
}

// Lays the workspace out; with base == nullptr only computes the size.
size_t plan_block(const hm_layer* L, int64_t T, int32_t k, int32_t lx, int32_t lz,
                  uint32_t flags, void* base, BlockPlan* p) {
    const int64_t H = L->hidden, I = L->intermediate, E = L->experts;
    const int64_t P = T * k;
    Carve c(base);
    BlockPlan q{};
    q.route_ws = c.take<char>(hm_route_workspace_bytes(T, L->hidden, E));
    q.permute_ws = c.take<char>(hm_permute_workspace_bytes(T, k, E));
    q.ids = c.take<uint32_t>((size_t)P);
    q.scores = c.take<float>((size_t)P);
    q.counts = c.take<int32_t>((size_t)E);
    q.offsets = c.take<int32_t>((size_t)E + 1);
    q.perm_tokens = c.take<int32_t>((size_t)P);
    q.perm_weights = c.take<float>((size_t)P);
    q.slots = c.take<int32_t>((size_t)P);
    q.status = c.take<int32_t>(1);
    if (use_gemv(L, T, k, flags)) {
        q.zf = c.take<float>((size_t)P * I);
        q.counters = c.take<int32_t>(1);
    } else if (L->dtype == HM_DTYPE_INT8) {
        q.xdig = c.take<int8_t>((size_t)lx * T * hm_pad64(H));  // X layout (hm_dlay_x)
        q.xscale = c.take<float>((size_t)T);
        q.xdsum = c.take<int32_t>((size_t)lx * T);
        q.zdig = c.take<int8_t>((size_t)lz * P * hm_pad64(I));  // Z layout (hm_dlay_z)
        q.zscale = c.take<float>((size_t)P);
        q.zdsum = c.take<int32_t>((size_t)lz * P);
        // the gate/up values [P x 2I] are dead once the Z digits are cut,
        // before the down projection writes y: one region serves both
        q.y = c.take<float>((size_t)P * (H > 2 * I ? H : 2 * I));
        q.gu = q.y;
        // decode batches: the fused router's completion counter
        if (T <= HM_GEMV_MAX_TOKENS) q.counters = c.take<int32_t>(1);
        if (p) *p = q;
        return c.used;
    } else {
        q.zf = c.take<float>((size_t)P * I);
        // FP32 decode batches: the fused router's completion counter too
        if (T <= HM_GEMV_MAX_TOKENS) q.counters = c.take<int32_t>(1);
    }
    q.y = c.take<float>((size_t)P * H);
    if (p) *p = q;
    return c.used;
}

}  // namespace


extern "C" {

size_t hm_moe_block_workspace_bytes(const hm_layer* layer, int64_t tokens, int32_t top_k,
                                    int32_t limbs_x, int32_t limbs_z, uint32_t exec_flags) {
    if (!layer_valid(layer) || tokens <= 0 || top_k <= 0) return 0;
    return plan_block(layer, tokens, top_k, limbs_x, limbs_z, exec_flags, nullptr, nullptr) +
           kAlign;
}

}  // extern "C"

namespace {

// The layer's RMSNorm ahead of the block (hm_moe_layer_forward): h is the
// layer input and the residual, normed receives RMSNorm(h).
struct LayerNorm {
    const float* gamma;
    float eps;
    float* normed;
};

// hm_moe_block_forward, and with `ln` the RMSNorm before it (folded into
// the decode router's first kernel, else its own launch).
int block_forward(const hm_layer* layer, const float* hidden, const float* router_w,
                  int64_t tokens, int32_t top_k, uint32_t route_flags, int32_t limbs_x,
                  int32_t limbs_z, const hm_block_io* io_in, void* workspace,
                  size_t workspace_bytes, void* stream, const LayerNorm* ln) {
    HM_REQUIRE(layer_valid(layer) && hidden && router_w && io_in && io_in->out && workspace);
    hm_block_io io_ln;
    const hm_block_io* io = io_in;
    if (ln) {
        // h is the residual; normed is read by every kernel after the norm
        // while h is still read, so the two must not overlap
        HM_REQUIRE(ln->gamma && ln->normed && std::isfinite(ln->eps) && ln->eps > 0.0f);
        HM_REQUIRE(!io_in->residual || io_in->residual == hidden);
        const size_t row_bytes = (size_t)layer->hidden * sizeof(float);
        const uintptr_t a0 = reinterpret_cast<uintptr_t>(hidden),
                        b0 = reinterpret_cast<uintptr_t>(ln->normed);
        HM_REQUIRE(tokens <= 0 || a0 + (size_t)tokens * row_bytes <= b0 ||
                   b0 + (size_t)tokens * row_bytes <= a0);
        io_ln = *io_in;
        io_ln.residual = hidden;
        io = &io_ln;
    }
    HM_REQUIRE(tokens > 0 && top_k > 0 && top_k <= layer->experts);
    if (layer->dtype == HM_DTYPE_INT8) {
        HM_REQUIRE(limbs_x >= 1 && limbs_x <= 3 && limbs_z >= 1 && limbs_z <= 3);
        if (layer->hidden > 65536 || layer->intermediate > 65536) return HM_ERR_OVERFLOW;
    }
    if (tokens > INT_MAX / top_k) return HM_ERR_OVERFLOW;
    const bool generic = (route_flags & HM_EXEC_GENERIC) != 0;
    const bool split_k = (route_flags & HM_EXEC_SPLIT_K) != 0;
    void* base = reinterpret_cast<void*>(
        (reinterpret_cast<uintptr_t>(workspace) + kAlign - 1) & ~(uintptr_t)(kAlign - 1));
    const size_t need =
        plan_block(layer, tokens, top_k, limbs_x, limbs_z, route_flags, nullptr, nullptr);
    HM_REQUIRE(workspace_bytes >= need + (size_t)(static_cast<char*>(base) - static_cast<char*>(workspace)));
    BlockPlan p;
    plan_block(layer, tokens, top_k, limbs_x, limbs_z, route_flags, base, &p);
    const bool gemv = use_gemv(layer, tokens, top_k, route_flags);
    if (io->ids) p.ids = io->ids;
    if (io->scores) p.scores = io->scores;
    if (io->counts) p.counts = io->counts;
    if (io->offsets) p.offsets = io->offsets;
    if (io->perm_tokens) p.perm_tokens = io->perm_tokens;
    if (io->perm_weights) p.perm_weights = io->perm_weights;
    if (io->expert_out) p.y = io->expert_out;
    int32_t* status = io->status ? io->status : p.status;
    hipStream_t s = hm_stream(stream);
    hipEvent_t ev[HM_BLOCK_EVENTS] = {};
    if (io->events) {
        for (int i = 0; i < HM_BLOCK_EVENTS; ++i) ev[i] = static_cast<hipEvent_t>(io->events[i]);
    }
    auto mark = [&](int i) -> int {
        if (ev[i]) HM_HIP(hipEventRecord(ev[i], s));
        return HM_OK;
    };
    int rc = mark(0);
    if (rc) return rc;
    if (!io->status) {
        hipLaunchKernelGGL(zero_status_kernel, dim3(1), dim3(1), 0, s, status);
        HM_LAUNCHED();
    }
    const int64_t E = layer->experts, H = layer->hidden;
    const int64_t P = tokens * top_k;
    const uint32_t route_bits =
        route_flags & (HM_ROUTE_SOFTMAX | HM_ROUTE_RENORM | HM_EXEC_ROUTE_SEQUENTIAL);
    // decode: the grouping is fused into the router's select (one launch
    // fewer)
    // FP32 experts of a decode batch take the FP32 GEMV (its rows are the
    // normalised ones when the layer's RMSNorm runs first, so their
    // alignment is the one that decides)
    const void* gemv_rows = ln ? static_cast<const void*>(ln->normed) : static_cast<const void*>(hidden);
    const bool gv32 = layer->dtype == HM_DTYPE_FP32 && tokens <= HM_GEMV_MAX_TOKENS &&
                      p.counters && hm_gemv_f32_ok(layer, gemv_rows) && hm_gemv_f32_ok(layer, p.zf);
    // INT8 decode batches on the limb GEMMs: the fused router also cuts the
    // activation digits
    const bool limb_decode = layer->dtype == HM_DTYPE_INT8 && !gemv &&
                             tokens <= HM_GEMV_MAX_TOKENS && p.counters && p.xdig;
    const bool fuse = (gemv || gv32 || limb_decode) && H % 32 == 0 && E <= 1024 && top_k <= 64 &&
                      P <= 1024;
    bool x_quantized = false;
    // one token on the GEMV path: the select runs inside the gate/up launch
    // (select_gateup_kernel), after the router partials
    const bool sel_gu = gemv && fuse && tokens == 1 && hm_select_gateup_ok(layer, top_k);
    if (fuse) {
        const hm_decode_fusion f = {p.counters, 1, p.counts, p.offsets, p.perm_tokens,
                                    p.perm_weights, p.slots};
        const hm_norm_fold nf = {ln ? ln->gamma : nullptr, ln ? ln->normed : nullptr,
                                 ln ? ln->eps : 0.0f,
                                 (route_flags & HM_EXEC_ROUTE_SEQUENTIAL) ? 1 : 0};
        const hm_row_quant xq = {p.xdig, p.xscale, p.xdsum, limbs_x};
        rc = sel_gu ? hm_route_partials_decode(hidden, router_w, H, E, top_k, route_bits, status,
                                               p.route_ws, &f, ln ? &nf : nullptr, stream)
                    : hm_route_permute_decode(hidden, router_w, tokens, H, E, top_k, route_bits,
                                              p.ids, p.scores, status, p.route_ws, &f,
                                              ln ? &nf : nullptr, limb_decode ? &xq : nullptr,
                                              &x_quantized, stream);
        if (ln) hidden = ln->normed;
        if (rc || (rc = mark(1)) || (rc = mark(2))) return rc;
    } else {
        if (ln) {
            rc = hm_launch_rmsnorm(hidden, ln->gamma, ln->normed, tokens, H, ln->eps,
                                   (route_flags & HM_EXEC_ROUTE_SEQUENTIAL) != 0, stream);
            if (rc) return rc;
            hidden = ln->normed;
        }
        // the INT8 expert path's activation digits come out of the router's
        // prefill select kernel when it runs (one launch fewer)
        const hm_row_quant xq = {p.xdig, p.xscale, p.xdsum, limbs_x};
        const bool want_q = !gemv && layer->dtype == HM_DTYPE_INT8 && p.xdig;
        // and the permutation's chunk histograms (its count pass) as well
        bool counted = false;
        rc = hm_router_topk_quant(hidden, router_w, tokens, H, E, top_k, route_bits, p.ids,
                                  p.scores, nullptr, status, p.route_ws, want_q ? &xq : nullptr,
                                  &x_quantized, reinterpret_cast<int32_t*>(p.permute_ws),
                                  &counted, stream);
        if (rc || (rc = mark(1))) return rc;
        rc = hm_permute_counted(p.ids, p.scores, tokens, top_k, E, p.counts, p.offsets,
                                p.perm_tokens, p.perm_weights, p.slots, p.permute_ws, counted,
                                stream);
        if (rc || (rc = mark(2))) return rc;
    }
    const int32_t* counts = p.counts;
    // The gate/up stage's two events are taken by its own kernels (start of
    // the first, end of the last) rather than by markers around them.
    const bool kernel_timed = ev[3] && ev[4];
    auto gate_up = [&](auto&& launch) -> int {
        if (!kernel_timed) {
            const int r = mark(3);
            if (r) return r;
        } else {
            hm_timer() = {ev[3], ev[4]};
        }
        const int r = launch();
        hm_timer() = {nullptr, nullptr};
        return r ? r : (kernel_timed ? HM_OK : mark(4));
    };
    if (gemv) {
        rc = gate_up([&] {
            return sel_gu ? hm_launch_select_gateup(hidden, router_w, top_k, route_bits, p.ids,
                                                    p.scores, status, p.route_ws, p.counts,
                                                    p.offsets, p.perm_tokens, p.perm_weights,
                                                    p.slots, layer, p.zf, s)
                          : hm_launch_gateup_gemv(layer, hidden, counts, p.offsets, p.perm_tokens,
                                                  tokens, P, p.zf, s);
        });
        if (rc) return rc;
        // one or two tokens: the down projection and the combine in one
        // launch (the combine's events mark its end)
        if (E <= 1024 && hm_gemv_combine_ok(tokens, top_k, H, layer->intermediate)) {
            rc = hm_launch_down_combine_gemv(layer, p.zf, counts, p.ids, p.slots, p.scores,
                                             io->residual, tokens, top_k, io->expert_out,
                                             io->out, s);
            if (rc || (rc = mark(5)) || (rc = mark(6))) return rc;
            return HM_OK;
        }
        rc = hm_launch_down_gemv(layer, p.zf, counts, p.offsets, P, p.y, s);
    } else if (layer->dtype == HM_DTYPE_INT8) {
        if (!x_quantized) {
            rc = hm_launch_quantize_rows(hidden, tokens, H, limbs_x, p.xdig, p.xscale, p.xdsum, s);
            if (rc) return rc;
        }
        rc = gate_up([&] {
            return hm_launch_gateup_i8(layer, limbs_x, limbs_z, p.xdig, p.xscale, p.xdsum,
                                       tokens, counts, p.offsets, p.perm_tokens, P, p.zdig,
                                       p.zscale, p.zdsum, p.gu, generic, split_k, s);
        });
        if (rc) return rc;
        rc = hm_launch_down_i8(layer, limbs_x, limbs_z, counts, p.offsets, P, p.zdig,
                               p.zscale, p.zdsum, p.y, generic, split_k, s);
    } else {
        // FP32 experts: decode-size batches stream each selected expert's
        // rows once (GEMV); others take the matrix-core tiles
        rc = gate_up([&] {
            return gv32 ? hm_launch_gateup_gemv_f32(layer, hidden, counts, p.offsets,
                                                    p.perm_tokens, P, p.zf, s)
                        : hm_launch_gateup_f32(layer, hidden, counts, p.offsets, p.perm_tokens,
                                               P, p.zf, s);
        });
        if (rc) return rc;
        rc = gv32 ? hm_launch_down_gemv_f32(layer, p.zf, counts, p.offsets, P, p.y, s)
                  : hm_launch_down_f32(layer, counts, p.offsets, P, p.zf, p.y, s);
    }
    if (rc || (rc = mark(5))) return rc;
    rc = hm_combine(p.y, p.ids, p.slots, p.scores, tokens, top_k, H, io->residual, io->out,
                    stream);
    if (rc || (rc = mark(6))) return rc;
    return HM_OK;
}

}  // namespace

extern "C" {

int hm_moe_block_forward(const hm_layer* layer, const float* hidden, const float* router_w,
                         int64_t tokens, int32_t top_k, uint32_t route_flags,
                         int32_t limbs_x, int32_t limbs_z, const hm_block_io* io,
                         void* workspace, size_t workspace_bytes, void* stream) {
    return block_forward(layer, hidden, router_w, tokens, top_k, route_flags, limbs_x, limbs_z,
                         io, workspace, workspace_bytes, stream, nullptr);
}

int hm_moe_layer_forward(const hm_layer* layer, const float* h, const float* gamma, float eps,
                         float* normed, const float* router_w, int64_t tokens, int32_t top_k,
                         uint32_t route_flags, int32_t limbs_x, int32_t limbs_z,
                         const hm_block_io* io, void* workspace, size_t workspace_bytes,
                         void* stream) {
    const LayerNorm ln = {gamma, eps, normed};
    return block_forward(layer, h, router_w, tokens, top_k, route_flags, limbs_x, limbs_z, io,
                         workspace, workspace_bytes, stream, &ln);
}

}  // extern "C"

extern "C" {

// Quantization.cpp:45-79 on the host: the reference's deterministic
// per-projection affine packer (scale = max|w|/127, zp = 0, round half away
// from zero, clamp to [-127, 127]).
int hm_quantize_int8_host(const float* w, int64_t n, int8_t* q, float* scale,
                          int32_t* zero_point, float* max_abs_error) {
    HM_REQUIRE(w && q && scale && zero_point && n > 0);
    float maximum = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        if (!std::isfinite(w[i])) return HM_ERR_INVALID;
        const float m = fabsf(w[i]);
        if (m > maximum) maximum = m;
    }
    const float s = maximum == 0.0f ? 1.0f : maximum / 127.0f;
    float err = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        float r = roundf(w[i] / s);
        r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
        q[i] = (int8_t)r;
        const float rec = (float)(int32_t)q[i] * s;
        const float d = fabsf(w[i] - rec);
        if (d > err) err = d;
    }
    *scale = s;
    *zero_point = 0;
    if (max_abs_error) *max_abs_error = err;
    return HM_OK;
}

}  // extern "C"
