// hm_router.hip -- RMSNorm, router top-k, token permute, gather, combine and
// elementwise kernels for gfx950 (wave64).  Every kernel here reproduces the
// reference CPU arithmetic bit for bit; the comments say how.
#include "hm_device.h"

#include <limits.h>

namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ void hm_status_or(int32_t* status, unsigned bits) {
    if (status) atomicOr(reinterpret_cast<unsigned int*>(status), bits);
}

// ---------------------------------------------------------------------------
// A1 RMSNorm (src/transformer/norm/RMSNorm.cpp:65-77), one workgroup per row.
//
// The reference sums double(x)^2 sequentially.  Squares of floats are exact
// in double, so only the summation order differs between a tree sum s_fast
// and the sequential s_seq; both lie within gamma_{n-1} * S of the exact sum
// S (any recursive summation order, Higham eq. 4.4), so
//   s_seq in [s_fast (1 - d), s_fast (1 + d)],  d = 4 gamma_{n-1}/(1-gamma).
// inv(s) = 1/sqrt(s/W + eps) and y(inv) = float(x * inv * g) are monotone
// under IEEE rounding, so an element whose y is equal at both ends of the
// interval equals the reference's y.  If any element of the row is
// ambiguous, the row falls back to the sequential sum (thread 0), which is
// the reference computation itself.
// ---------------------------------------------------------------------------
__device__ __forceinline__ double hm_inv_rms(double s, double width, double eps) {
    return 1.0 / sqrt(s / width + eps);
}

__global__ __launch_bounds__(kBlock) void rmsnorm_kernel(
    const float* __restrict__ x, const float* __restrict__ gamma,
    float* __restrict__ y, int64_t width, float eps) {
    extern __shared__ float row_lds[];  // width floats
    __shared__ double red[kBlock / HM_WAVE];
    __shared__ int ambiguous;
    __shared__ double inv_seq;
    const int64_t r = blockIdx.x;
    const float* xr = x + r * width;
    float* yr = y + r * width;
    const int tid = threadIdx.x;
    if (tid == 0) ambiguous = 0;
    double local = 0.0;
    for (int64_t i = tid; i < width; i += kBlock) {
        const float v = xr[i];
        row_lds[i] = v;
        local += (double)v * v;
    }
    local = hm_wave_sum_f64(local);
    if ((tid & (HM_WAVE - 1)) == 0) red[tid / HM_WAVE] = local;
    __syncthreads();
    double s_fast = 0.0;
    for (int w = 0; w < kBlock / HM_WAVE; ++w) s_fast += red[w];
    const double u = 0x1p-53;
    const double gam = (double)(width - 1) * u / (1.0 - (double)(width - 1) * u);
    const double d = 4.0 * gam / (1.0 - gam);
    const double wd = (double)width, ed = (double)eps;
    const double inv_lo = hm_inv_rms(s_fast * (1.0 + d), wd, ed);
    const double inv_hi = hm_inv_rms(s_fast * (1.0 - d), wd, ed);
    for (int64_t i = tid; i < width; i += kBlock) {
        const float v = row_lds[i];
        const float a = (float)((double)v * inv_lo * (double)gamma[i]);
        const float b = (float)((double)v * inv_hi * (double)gamma[i]);
        if (__float_as_uint(a) == __float_as_uint(b)) {
            yr[i] = a;
        } else {
            ambiguous = 1;
        }
    }
    __syncthreads();
    if (!ambiguous) return;
    if (tid == 0) {
        double s = 0.0;
        for (int64_t i = 0; i < width; ++i) {
            const float v = row_lds[i];
            s += (double)v * v;
        }
        inv_seq = hm_inv_rms(s, wd, ed);
    }
    __syncthreads();
    const double inv = inv_seq;
    for (int64_t i = tid; i < width; i += kBlock) {
        yr[i] = (float)((double)row_lds[i] * inv * (double)gamma[i]);
    }
}

// ---------------------------------------------------------------------------
// A2 router logits (src/router/CpuRouterBackend.cpp:41-49):
//   logit[t,e] = float(sum_k double(h[t,k]) * double(w[k,e])), k ascending.
// The product of two floats is exact in double, so fma(h, w, acc) rounds
// exactly like the reference's multiply-then-add: each lane owns (t, e)
// pairs and runs the k loop in order.  Tiles: 32 tokens x 64 experts per
// workgroup, k staged through LDS as doubles; lane = expert, each wave owns
// 8 tokens (8 independent FMA chains per lane).
// Also zeroes the routing bitmask and per-expert counts for the select pass.
// ---------------------------------------------------------------------------
constexpr int kLogitTokens = 32;
constexpr int kLogitExperts = 64;
constexpr int kLogitK = 32;

__global__ __launch_bounds__(kBlock) void router_logits_kernel(
    const float* __restrict__ h, const float* __restrict__ w, int64_t tokens,
    int64_t hidden, int64_t experts, float* __restrict__ logits,
    int32_t* status, uint32_t* __restrict__ zero_words, int64_t zero_count) {
    __shared__ double hs[kLogitTokens][kLogitK + 1];
    __shared__ double ws[kLogitK][kLogitExperts];
    const int tid = threadIdx.x;
    {   // clear the routing bitmask + counts (grid-stride)
        const int64_t nthreads = (int64_t)gridDim.x * gridDim.y * kBlock;
        const int64_t gid = ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * kBlock + tid;
        for (int64_t i = gid; i < zero_count; i += nthreads) zero_words[i] = 0u;
    }
    const int lane = tid & (HM_WAVE - 1);
    const int wave = tid / HM_WAVE;
    const int64_t t0 = (int64_t)blockIdx.x * kLogitTokens;
    const int64_t e0 = (int64_t)blockIdx.y * kLogitExperts;
    double acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0;
    for (int64_t k0 = 0; k0 < hidden; k0 += kLogitK) {
        for (int i = tid; i < kLogitTokens * kLogitK; i += kBlock) {
            const int tt = i / kLogitK, kk = i % kLogitK;
            const int64_t t = t0 + tt, k = k0 + kk;
            hs[tt][kk] = (t < tokens && k < hidden) ? (double)h[t * hidden + k] : 0.0;
        }
        for (int i = tid; i < kLogitK * kLogitExperts; i += kBlock) {
            const int kk = i / kLogitExperts, ee = i % kLogitExperts;
            const int64_t k = k0 + kk, e = e0 + ee;
            ws[kk][ee] = (k < hidden && e < experts) ? (double)w[k * experts + e] : 0.0;
        }
        __syncthreads();
        const int kn = (int)((hidden - k0) < kLogitK ? (hidden - k0) : kLogitK);
        for (int kk = 0; kk < kn; ++kk) {
            const double wv = ws[kk][lane];
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] = __builtin_fma(hs[wave * 8 + i][kk], wv, acc[i]);
        }
        __syncthreads();
    }
    const int64_t e = e0 + lane;
    if (e >= experts) return;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int64_t t = t0 + wave * 8 + i;
        if (t >= tokens) break;
        if (!isfinite(acc[i])) hm_status_or(status, HM_STATUS_NONFINITE_SCORE);
        logits[t * experts + e] = (float)acc[i];
    }
}

// ---------------------------------------------------------------------------
// A2 select (src/router/CpuRouterBackend.cpp:50-89), one wave per token.
//   softmax: m = max logit; p = expf(l - m) (float, glibc-exact hm_expf);
//            den = sum_e double(p) in ascending e; p = float(double(p)/den).
//   The sum: every p is in [0, 1] and p(max) = 1, so den < 2^12 for
//   E <= 2048.  If every nonzero p is >= 2^-17 its last bit is >= 2^-40,
//   every partial sum is a multiple of 2^-40 below 2^13 and hence exact in
//   double, so any order gives the sequential result; otherwise lane 0 sums
//   sequentially.
//   top-k: k rounds of a wave argmax over hm_rank_key (score desc, id asc),
//   i.e. std::partial_sort with the reference comparator.
//   renorm: sum of the k selected scores in rank order in double.
// Writes ids/scores [t, r] in rank order, sets bit t of row e of the routing
// bitmask and counts[e] += 1 for every selected e.
// ---------------------------------------------------------------------------
template <int EPL>
__global__ __launch_bounds__(kBlock) void router_select_kernel(
    const float* __restrict__ logits, int64_t tokens, int64_t experts,
    int32_t top_k, uint32_t flags, uint32_t* __restrict__ ids,
    float* __restrict__ scores, uint32_t* __restrict__ mask, int64_t mask_words,
    int32_t* __restrict__ counts, int32_t* status) {
    extern __shared__ float seq_lds[];  // (kBlock/64) * experts floats
    const int lane = threadIdx.x & (HM_WAVE - 1);
    const int wave = threadIdx.x / HM_WAVE;
    const int64_t t = (int64_t)blockIdx.x * (kBlock / HM_WAVE) + wave;
    if (t >= tokens) return;
    const float* lt = logits + t * experts;
    float v[EPL];
    bool valid[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        const int64_t e = lane + (int64_t)HM_WAVE * j;
        valid[j] = e < experts;
        v[j] = valid[j] ? lt[e] : 0.0f;
    }
    if (flags & HM_ROUTE_SOFTMAX) {
        float m = -__uint_as_float(0x7f800000u);
#pragma unroll
        for (int j = 0; j < EPL; ++j) if (valid[j]) m = fmaxf(m, v[j]);
        m = hm_wave_max_f32(m);
        bool exact = true;
        double part = 0.0;
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            if (!valid[j]) continue;
            v[j] = hm_expf(__fsub_rn(v[j], m));
            exact = exact && (v[j] == 0.0f || v[j] >= 0x1p-17f);
            part += (double)v[j];
        }
        double den;
        if (__all(exact) && experts <= 2048) {
            den = hm_wave_sum_f64(part);
        } else {
            float* seq = seq_lds + (int64_t)wave * experts;
#pragma unroll
            for (int j = 0; j < EPL; ++j) if (valid[j]) seq[lane + HM_WAVE * j] = v[j];
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            double s = 0.0;
            if (lane == 0) for (int64_t e = 0; e < experts; ++e) s += (double)seq[e];
            den = __shfl(s, 0, HM_WAVE);
        }
        if (!(isfinite(den) && den > 0.0)) {
            if (lane == 0) hm_status_or(status, HM_STATUS_SOFTMAX_FAILED);
            return;
        }
#pragma unroll
        for (int j = 0; j < EPL; ++j) if (valid[j]) v[j] = (float)((double)v[j] / den);
    }
    unsigned long long key[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        key[j] = valid[j] ? hm_rank_key(v[j], (unsigned)(lane + HM_WAVE * j)) : 0ull;
    }
    uint32_t my_id = 0;
    float my_score = 0.0f;
    double sel_sum = 0.0;
    for (int r = 0; r < top_k; ++r) {
        unsigned long long best = 0ull;
#pragma unroll
        for (int j = 0; j < EPL; ++j) best = key[j] > best ? key[j] : best;
        best = hm_wave_max_u64(best);
        const uint32_t id = 0xffffffffu - (uint32_t)(best & 0xffffffffull);
        const int owner = (int)(id % HM_WAVE);
        const int slot = (int)(id / HM_WAVE);
        float sv = 0.0f;
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            if (j == slot && lane == owner) { sv = v[j]; key[j] = 0ull; }
        }
        sv = __shfl(sv, owner, HM_WAVE);
        sel_sum += (double)sv;  // rank order, uniform across lanes
        if (lane == r) { my_id = id; my_score = sv; }
    }
    if (flags & HM_ROUTE_RENORM) {
        if (!(isfinite(sel_sum) && sel_sum != 0.0)) {
            if (lane == 0) hm_status_or(status, HM_STATUS_RENORM_FAILED);
            return;
        }
        my_score = (float)((double)my_score / sel_sum);
    }
    if (lane < top_k) {
        ids[t * top_k + lane] = my_id;
        scores[t * top_k + lane] = my_score;
        atomicOr(&mask[(int64_t)my_id * mask_words + (t >> 5)], 1u << (t & 31));
        atomicAdd(&counts[my_id], 1);
    }
}

// ---------------------------------------------------------------------------
// A3 permute (src/router/CpuRouterBackend.cpp:140-159): one workgroup per
// expert.  Bit t of row e is set iff token t selected e; scanning the row in
// ascending t gives the reference's group order (tokens ascending), and
// offsets[e] = sum of counts of lower ids gives groups in ascending id.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void permute_kernel(
    const uint32_t* __restrict__ ids, const float* __restrict__ scores,
    int64_t tokens, int32_t top_k, int64_t experts,
    const uint32_t* __restrict__ mask, int64_t mask_words,
    const int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ perm_tokens, float* __restrict__ perm_weights,
    int32_t* __restrict__ slots) {
    __shared__ int red[kBlock];
    const int tid = threadIdx.x;
    const int64_t e = blockIdx.x;
    int part = 0;
    for (int64_t i = tid; i < e; i += kBlock) part += counts[i];
    red[tid] = part;
    __syncthreads();
    for (int s = kBlock / 2; s > 0; s >>= 1) {
        if (tid < s) red[tid] += red[tid + s];
        __syncthreads();
    }
    const int offset = red[0];
    __syncthreads();
    if (tid == 0) {
        offsets[e] = offset;
        if (e == experts - 1) offsets[experts] = offset + counts[e];
    }
    const uint32_t* row = mask + e * mask_words;
    const int64_t chunk = (mask_words + kBlock - 1) / kBlock;
    const int64_t w_begin = tid * chunk;
    const int64_t w_end = (w_begin + chunk) < mask_words ? (w_begin + chunk) : mask_words;
    int mine = 0;
    for (int64_t wi = w_begin; wi < w_end; ++wi) mine += __popc(row[wi]);
    red[tid] = mine;
    __syncthreads();
    // inclusive Hillis-Steele scan over 256 entries
    for (int s = 1; s < kBlock; s <<= 1) {
        const int add = tid >= s ? red[tid - s] : 0;
        __syncthreads();
        red[tid] += add;
        __syncthreads();
    }
    int pos = offset + red[tid] - mine;
    for (int64_t wi = w_begin; wi < w_end; ++wi) {
        uint32_t bits = row[wi];
        while (bits) {
            const int b = __ffs(bits) - 1;
            bits &= bits - 1;
            const int64_t t = wi * 32 + b;
            int r = 0;
            for (; r < top_k; ++r) if (ids[t * top_k + r] == (uint32_t)e) break;
            perm_tokens[pos] = (int32_t)t;
            if (r < top_k) {
                perm_weights[pos] = scores[t * top_k + r];
                slots[t * top_k + r] = pos;
            }
            ++pos;
        }
    }
}

// A4 gather (MoERuntime.cpp:288-298).
__global__ void gather_rows_kernel(const float* __restrict__ in,
                                   const int32_t* __restrict__ rows,
                                   int64_t count, int64_t width,
                                   float* __restrict__ out) {
    const int64_t r = blockIdx.y;
    const float* src = in + (int64_t)rows[r] * width;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < width;
         i += (int64_t)gridDim.x * kBlock) {
        out[r * width + i] = src[i];
    }
}

// ---------------------------------------------------------------------------
// A7 combine (src/core/runtime/MoERuntime.cpp:312-324): per token, the
// reference adds w * y over groups in ascending expert id, starting from 0,
// with a separate float multiply and add.  The k selected ids of a token are
// distinct, so sorting them gives that order.  Optional residual added last
// (TransformerBlock.cpp:101-104).
// ---------------------------------------------------------------------------
constexpr int kMaxTopK = 64;

__global__ __launch_bounds__(kBlock) void combine_kernel(
    const float* __restrict__ y, const uint32_t* __restrict__ ids,
    const int32_t* __restrict__ slots, const float* __restrict__ scores,
    int64_t tokens, int32_t top_k, int64_t width,
    const float* __restrict__ residual, float* __restrict__ out) {
    __shared__ int64_t srow[kMaxTopK];
    __shared__ float sw[kMaxTopK];
    const int64_t t = blockIdx.y;
    if (threadIdx.x == 0) {
        // insertion sort of the (id, slot, weight) triples by id
        uint32_t sid[kMaxTopK];
        for (int r = 0; r < top_k; ++r) {
            const uint32_t id = ids[t * top_k + r];
            const int64_t row = slots[t * top_k + r];
            const float wv = scores[t * top_k + r];
            int j = r;
            while (j > 0 && sid[j - 1] > id) {
                sid[j] = sid[j - 1];
                srow[j] = srow[j - 1];
                sw[j] = sw[j - 1];
                --j;
            }
            sid[j] = id;
            srow[j] = row;
            sw[j] = wv;
        }
    }
    __syncthreads();
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < width;
         i += (int64_t)gridDim.x * kBlock) {
        float acc = 0.0f;
        for (int r = 0; r < top_k; ++r) {
            acc = __fadd_rn(acc, __fmul_rn(sw[r], y[srow[r] * width + i]));
        }
        if (residual) acc = __fadd_rn(residual[t * width + i], acc);
        out[t * width + i] = acc;
    }
}

// A6 elementwise (Activation.cpp:44, CpuTensorBackend.cpp:202-204, 217-219).
__global__ void silu_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kBlock) y[i] = hm_silu(x[i]);
}
__global__ void mul_kernel(const float* __restrict__ a, const float* __restrict__ b,
                           float* __restrict__ y, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kBlock) y[i] = __fmul_rn(a[i], b[i]);
}
__global__ void add_kernel(const float* __restrict__ a, const float* __restrict__ b,
                           float* __restrict__ y, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kBlock) y[i] = __fadd_rn(a[i], b[i]);
}
__global__ void expf_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kBlock) y[i] = hm_expf(x[i]);
}

unsigned grid_for(int64_t n) {
    int64_t g = (n + kBlock - 1) / kBlock;
    if (g < 1) g = 1;
    if (g > 65535) g = 65535;
    return (unsigned)g;
}

}  // namespace

// Route workspace layout: logits [T x E] f32 | mask [E x ceil(T/32)] u32 |
// counts [E] i32.
static int64_t mask_words_for(int64_t tokens) { return (tokens + 31) / 32; }

int32_t* hm_route_counts_ptr(void* route_ws, int64_t tokens, int64_t experts) {
    char* ws = static_cast<char*>(route_ws);
    const size_t logit_bytes = ((size_t)tokens * experts * sizeof(float) + 255) & ~(size_t)255;
    uint32_t* mask = reinterpret_cast<uint32_t*>(ws + logit_bytes);
    return reinterpret_cast<int32_t*>(mask + experts * mask_words_for(tokens));
}

extern "C" {

int hm_rmsnorm(const float* x, const float* gamma, float* y, int64_t rows,
               int64_t width, float eps, void* stream) {
    HM_REQUIRE(x && gamma && y && rows >= 0 && width > 0);
    HM_REQUIRE(std::isfinite(eps) && eps > 0.0f);  // RMSNorm.cpp:22
    HM_REQUIRE(width <= 16384);              // row staged in LDS
    if (rows == 0) return HM_OK;
    HM_REQUIRE(rows <= INT_MAX);
    hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(kBlock),
                       (size_t)width * sizeof(float), hm_stream(stream), x, gamma,
                       y, width, eps);
    HM_LAUNCHED();
    return HM_OK;
}

size_t hm_route_workspace_bytes(int64_t tokens, int64_t experts) {
    if (tokens < 0 || experts <= 0) return 0;
    const size_t logits = (size_t)tokens * (size_t)experts * sizeof(float);
    const size_t mask = (size_t)experts * (size_t)mask_words_for(tokens) * sizeof(uint32_t);
    return ((logits + 255) & ~(size_t)255) + mask + (size_t)experts * sizeof(int32_t);
}

int hm_router_topk(const float* h, const float* w, int64_t tokens,
                   int64_t hidden, int64_t experts, int32_t top_k,
                   uint32_t flags, uint32_t* ids, float* scores,
                   float* logits_out, int32_t* status, void* route_ws,
                   void* stream) {
    // RouterConfig::validate (src/router/RouterConfig.cpp:9-22)
    HM_REQUIRE(experts > 0 && top_k > 0 && top_k <= experts);
    HM_REQUIRE(h && w && ids && scores && route_ws && tokens > 0 && hidden > 0);
    if (experts > 1024 || top_k > kMaxTopK) return HM_ERR_UNSUPPORTED;
    if (tokens > ((int64_t)1 << 31) / kLogitTokens) return HM_ERR_OVERFLOW;
    const int64_t mw = mask_words_for(tokens);
    char* ws = static_cast<char*>(route_ws);
    const size_t logit_bytes = ((size_t)tokens * experts * sizeof(float) + 255) & ~(size_t)255;
    float* logits = logits_out ? logits_out : reinterpret_cast<float*>(ws);
    uint32_t* mask = reinterpret_cast<uint32_t*>(ws + logit_bytes);
    int32_t* counts = reinterpret_cast<int32_t*>(mask + experts * mw);
    const dim3 lgrid((unsigned)((tokens + kLogitTokens - 1) / kLogitTokens),
                     (unsigned)((experts + kLogitExperts - 1) / kLogitExperts));
    hipLaunchKernelGGL(router_logits_kernel, lgrid, dim3(kBlock), 0, hm_stream(stream),
                       h, w, tokens, hidden, experts, logits, status, mask,
                       experts * mw + experts);
    HM_LAUNCHED();
    const dim3 sgrid((unsigned)((tokens + 3) / 4));
    const size_t seq_bytes = (size_t)(kBlock / HM_WAVE) * experts * sizeof(float);
    const int epl = (int)((experts + HM_WAVE - 1) / HM_WAVE);
#define HM_SELECT(N)                                                                   \
    hipLaunchKernelGGL(router_select_kernel<N>, sgrid, dim3(kBlock), seq_bytes,        \
                       hm_stream(stream), logits, tokens, experts, top_k, flags, ids,  \
                       scores, mask, mw, counts, status)
    if (epl <= 1) HM_SELECT(1);
    else if (epl <= 2) HM_SELECT(2);
    else if (epl <= 4) HM_SELECT(4);
    else if (epl <= 8) HM_SELECT(8);
    else HM_SELECT(16);
#undef HM_SELECT
    HM_LAUNCHED();
    return HM_OK;
}

int hm_permute(const uint32_t* ids, const float* scores, int64_t tokens,
               int32_t top_k, int64_t experts, void* route_ws, int32_t* counts,
               int32_t* offsets, int32_t* perm_tokens, float* perm_weights,
               int32_t* slots, void* stream) {
    HM_REQUIRE(ids && scores && route_ws && offsets && perm_tokens && perm_weights && slots);
    HM_REQUIRE(tokens > 0 && top_k > 0 && experts > 0 && top_k <= experts);
    if (tokens * top_k > INT_MAX) return HM_ERR_OVERFLOW;
    const int64_t mw = mask_words_for(tokens);
    char* ws = static_cast<char*>(route_ws);
    const size_t logit_bytes = ((size_t)tokens * experts * sizeof(float) + 255) & ~(size_t)255;
    const uint32_t* mask = reinterpret_cast<const uint32_t*>(ws + logit_bytes);
    const int32_t* ws_counts = reinterpret_cast<const int32_t*>(mask + experts * mw);
    hipLaunchKernelGGL(permute_kernel, dim3((unsigned)experts), dim3(kBlock), 0,
                       hm_stream(stream), ids, scores, tokens, top_k, experts, mask,
                       mw, ws_counts, offsets, perm_tokens, perm_weights, slots);
    HM_LAUNCHED();
    if (counts) {
        HM_HIP(hipMemcpyAsync(counts, ws_counts, (size_t)experts * sizeof(int32_t),
                              hipMemcpyDeviceToDevice, hm_stream(stream)));
    }
    return HM_OK;
}

int hm_gather_rows(const float* in, const int32_t* rows, int64_t count,
                   int64_t width, float* out, void* stream) {
    HM_REQUIRE(in && rows && out && count >= 0 && width > 0);
    if (count == 0) return HM_OK;
    HM_REQUIRE(count <= 65535);
    const unsigned gx = (unsigned)((width + kBlock - 1) / kBlock > 64 ? 64 : (width + kBlock - 1) / kBlock);
    hipLaunchKernelGGL(gather_rows_kernel, dim3(gx, (unsigned)count), dim3(kBlock), 0,
                       hm_stream(stream), in, rows, count, width, out);
    HM_LAUNCHED();
    return HM_OK;
}

int hm_combine(const float* y_grouped, const uint32_t* ids, const int32_t* slots,
               const float* scores, int64_t tokens, int32_t top_k, int64_t width,
               const float* residual, float* out, void* stream) {
    HM_REQUIRE(y_grouped && ids && slots && scores && out);
    HM_REQUIRE(tokens > 0 && top_k > 0 && width > 0);
    if (top_k > kMaxTopK) return HM_ERR_UNSUPPORTED;
    HM_REQUIRE(tokens <= 65535);
    const unsigned gx = (unsigned)((width + kBlock - 1) / kBlock > 8 ? 8 : (width + kBlock - 1) / kBlock);
    hipLaunchKernelGGL(combine_kernel, dim3(gx, (unsigned)tokens), dim3(kBlock), 0,
                       hm_stream(stream), y_grouped, ids, slots, scores, tokens, top_k,
                       width, residual, out);
    HM_LAUNCHED();
    return HM_OK;
}

int hm_silu(const float* x, float* y, int64_t n, void* stream) {
    HM_REQUIRE(x && y && n >= 0);
    if (n == 0) return HM_OK;
    hipLaunchKernelGGL(silu_kernel, dim3(grid_for(n)), dim3(kBlock), 0, hm_stream(stream), x, y, n);
    HM_LAUNCHED();
    return HM_OK;
}

int hm_mul(const float* a, const float* b, float* y, int64_t n, void* stream) {
    HM_REQUIRE(a && b && y && n >= 0);
    if (n == 0) return HM_OK;
    hipLaunchKernelGGL(mul_kernel, dim3(grid_for(n)), dim3(kBlock), 0, hm_stream(stream), a, b, y, n);
    HM_LAUNCHED();
    return HM_OK;
}

int hm_add(const float* a, const float* b, float* y, int64_t n, void* stream) {
    HM_REQUIRE(a && b && y && n >= 0);
    if (n == 0) return HM_OK;
    hipLaunchKernelGGL(add_kernel, dim3(grid_for(n)), dim3(kBlock), 0, hm_stream(stream), a, b, y, n);
    HM_LAUNCHED();
    return HM_OK;
}

int hm_debug_expf(const float* x, float* y, int64_t n, void* stream) {
    HM_REQUIRE(x && y && n >= 0);
    if (n == 0) return HM_OK;
    hipLaunchKernelGGL(expf_kernel, dim3(grid_for(n)), dim3(kBlock), 0, hm_stream(stream), x, y, n);
    HM_LAUNCHED();
    return HM_OK;
}

}  // extern "C"
