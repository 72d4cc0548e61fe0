// hm_router.hip -- RMSNorm, router top-k, token permute, gather, combine and
// elementwise kernels for gfx950 (wave64).  Every kernel here reproduces the
// reference CPU arithmetic bit for bit; the comments say how.
#include "hm_device.h"
#include "hm_gemv_slice.h"
#include "hm_lds_dma.h"

#include <limits.h>

#include <type_traits>

namespace {

constexpr int kBlock = 256;
constexpr int kPermChunk = 1024;  // pairs per permutation chunk (kPermThreads)

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

// The relative half-width d of the interval around a tree sum of `width`
// squares that holds the sequential sum (above).
__device__ __forceinline__ double hm_rms_sum_slack(int64_t width) {
    const double u = 0x1p-53;
    const double gam = (double)(width - 1) * u / (1.0 - (double)(width - 1) * u);
    return 4.0 * gam / (1.0 - gam);
}

// The reference's own sum: double(x_k)^2 added in ascending k from +0
// (the values read 16 at a time, so that the reads overlap the additions).
__device__ __forceinline__ double hm_rms_sum_seq(const float* __restrict__ xr, int64_t width) {
    double s = 0.0;
    int64_t i = 0;
    for (; i + 16 <= width; i += 16) {
        float r[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) r[u] = xr[i + u];
#pragma unroll
        for (int u = 0; u < 16; ++u) s += (double)r[u] * r[u];
    }
    for (; i < width; ++i) {
        const float v = xr[i];
        s += (double)v * v;
    }
    return s;
}

__global__ __launch_bounds__(kBlock) void rmsnorm_kernel(
    const float* __restrict__ x, const float* __restrict__ gamma,
    float* __restrict__ y, int64_t width, float eps, int force_seq) {
    extern __shared__ float row_lds[];  // width floats
    __shared__ double red[kBlock / HM_WAVE];
    __shared__ int ambiguous;
    __shared__ double inv_seq;
    const int64_t r = blockIdx.x;
    const float* xr = x + r * width;
    float* yr = y + r * width;
    const int tid = threadIdx.x;
    if (tid == 0) ambiguous = force_seq;
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
    const double d = hm_rms_sum_slack(width);
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
    if (tid == 0) inv_seq = hm_inv_rms(hm_rms_sum_seq(row_lds, width), wd, ed);
    __syncthreads();
    const double inv = inv_seq;
    for (int64_t i = tid; i < width; i += kBlock) {
        yr[i] = (float)((double)row_lds[i] * inv * (double)gamma[i]);
    }
}

// The same RMSNorm for rows of 256 V floats (16-byte aligned), one wave per
// row and four rows per workgroup: a lane's V 16-byte loads are issued
// together and the row stays in registers (rmsnorm_kernel's strided loop
// waits for each load before the next).  Same bracket, same fallback (a row
// with an ambiguous element, or every row with force_seq, takes the
// sequential sum), with the exact
// products formed by the whole wave so that lane 0's chain is only the
// additions.
template <int V>
__global__ __launch_bounds__(kBlock) void rmsnorm_wave_kernel(
    const float* __restrict__ x, const float* __restrict__ gamma,
    float* __restrict__ y, int64_t rows, float eps, int force_seq) {
    constexpr int W = 256 * V;
    extern __shared__ float row_lds[];  // [4][512] doubles: a chunk of products per wave
    const int lane = threadIdx.x & (HM_WAVE - 1), wv = threadIdx.x / HM_WAVE;
    const int64_t r = (int64_t)blockIdx.x * (kBlock / HM_WAVE) + wv;
    if (r >= rows) return;
    const float4* xr = reinterpret_cast<const float4*>(x + r * W);
    const float4* g4 = reinterpret_cast<const float4*>(gamma);
    float4* yr = reinterpret_cast<float4*>(y + r * W);
    float4 v[V];
#pragma unroll
    for (int j = 0; j < V; ++j) v[j] = xr[HM_WAVE * j + lane];
    double local = 0.0;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        local += (double)v[j].x * v[j].x;
        local += (double)v[j].y * v[j].y;
        local += (double)v[j].z * v[j].z;
        local += (double)v[j].w * v[j].w;
    }
    const double s_fast = hm_wave_sum_f64(local);  // equal on every lane
    const double d = hm_rms_sum_slack(W);
    const double wd = (double)W, ed = (double)eps;
    const double inv_lo = hm_inv_rms(s_fast * (1.0 + d), wd, ed);
    const double inv_hi = hm_inv_rms(s_fast * (1.0 - d), wd, ed);
    float4 out[V];
    bool amb = false;
    auto one = [&](float xv, float gv, float& o) __attribute__((always_inline)) {
        const float a = (float)((double)xv * inv_lo * (double)gv);
        const float b = (float)((double)xv * inv_hi * (double)gv);
        o = a;
        amb |= __float_as_uint(a) != __float_as_uint(b);
    };
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const float4 g = g4[HM_WAVE * j + lane];
        one(v[j].x, g.x, out[j].x);
        one(v[j].y, g.y, out[j].y);
        one(v[j].z, g.z, out[j].z);
        one(v[j].w, g.w, out[j].w);
    }
    if (force_seq || __ballot(amb) != 0) {
        // The reference's sequential sum: s = fl(s + p_k) with the exact
        // products p_k = double(x_k)^2.  The wave forms the products of 512
        // consecutive elements (its registers j = 2q, 2q+1) into LDS, then
        // lane 0 adds them in order, 16 loaded ahead; the chain is one
        // dependent add per element.
        double* lp = reinterpret_cast<double*>(row_lds) + (int64_t)wv * 512;
        double s = 0.0;
#pragma unroll
        for (int q = 0; q < (V + 1) / 2; ++q) {
            const int nj = 2 * q + 1 < V ? 2 : 1;
#pragma unroll
            for (int jj = 0; jj < nj; ++jj) {
                const float4 x4 = v[2 * q + jj];
                double* d = lp + 256 * jj + 4 * lane;
                d[0] = (double)x4.x * x4.x;
                d[1] = (double)x4.y * x4.y;
                d[2] = (double)x4.z * x4.z;
                d[3] = (double)x4.w * x4.w;
            }
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
            if (lane == 0) {
                const double2* p2 = reinterpret_cast<const double2*>(lp);
                const int n2 = 128 * nj;  // pairs of products in this chunk
                double2 cur[8], nxt[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) cur[i] = p2[i];
                for (int b = 0; b < n2; b += 8) {
                    if (b + 8 < n2) {
#pragma unroll
                        for (int i = 0; i < 8; ++i) nxt[i] = p2[b + 8 + i];
                    }
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        s += cur[i].x;
                        s += cur[i].y;
                    }
#pragma unroll
                    for (int i = 0; i < 8; ++i) cur[i] = nxt[i];
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
        }
        double inv = 0.0;
        if (lane == 0) inv = hm_inv_rms(s, wd, ed);
        inv = __shfl(inv, 0, HM_WAVE);
#pragma unroll
        for (int j = 0; j < V; ++j) {
            const float4 g = g4[HM_WAVE * j + lane];
            out[j].x = (float)((double)v[j].x * inv * (double)g.x);
            out[j].y = (float)((double)v[j].y * inv * (double)g.y);
            out[j].z = (float)((double)v[j].z * inv * (double)g.z);
            out[j].w = (float)((double)v[j].w * inv * (double)g.w);
        }
    }
#pragma unroll
    for (int j = 0; j < V; ++j) yr[HM_WAVE * j + lane] = out[j];
}

// ---------------------------------------------------------------------------
// A2 router logits (src/router/CpuRouterBackend.cpp:41-49):
//   logit[t,e] = float(sum_k double(h[t,k]) * double(w[k,e])), k ascending.
// The product of two floats is exact in double, so fma(h, w, acc) rounds
// exactly like the reference's multiply-then-add, and each (t, e) chain runs
// k in order.  Workgroup tile: 16 tokens x 128 experts; thread (tt, te) owns
// tokens 2tt, 2tt+1 and experts 4te .. 4te+3 (8 independent FMA chains).
// k is staged through LDS as doubles in 32-wide chunks, double buffered, the
// next chunk prefetched into registers while the current one is consumed.
// ---------------------------------------------------------------------------
constexpr int kLT = 16;   // tokens per workgroup
constexpr int kLE = 128;  // experts per workgroup
constexpr int kLK = 32;   // k per chunk

__global__ __launch_bounds__(kBlock) void router_logits_kernel(
    const float* __restrict__ h, const float* __restrict__ w, int64_t tokens,
    int64_t hidden, int64_t experts, float* __restrict__ logits, int32_t* status) {
    __shared__ __attribute__((aligned(16))) double hs[2][kLK][kLT];
    __shared__ __attribute__((aligned(16))) double ws[2][kLK][kLE];
    const int tid = threadIdx.x;
    const int tt = tid >> 5, te = tid & 31;
    const int64_t t0 = (int64_t)blockIdx.x * kLT;
    const int64_t e0 = (int64_t)blockIdx.y * kLE;
    // staging: h chunk = 16 x 32 floats (2 per thread), w chunk = 32 x 128
    // floats (16 per thread, 4 groups of 4 consecutive experts).
    float hr[2], wr[4][4];
    auto fetch = [&](int64_t k0) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int idx = tid * 2 + c;
            const int t = idx / kLK, kk = idx % kLK;
            const int64_t tg = t0 + t, kg = k0 + kk;
            hr[c] = (tg < tokens && kg < hidden) ? h[tg * hidden + kg] : 0.0f;
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int idx = tid + kBlock * c;  // 0 .. 1023
            const int kk = idx >> 5, e4 = idx & 31;
            const int64_t kg = k0 + kk;
#pragma unroll
            for (int x = 0; x < 4; ++x) {
                const int64_t eg = e0 + 4 * e4 + x;
                wr[c][x] = (kg < hidden && eg < experts) ? w[kg * experts + eg] : 0.0f;
            }
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int idx = tid * 2 + c;
            hs[buf][idx % kLK][idx / kLK] = (double)hr[c];
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int idx = tid + kBlock * c;
            const int kk = idx >> 5, e4 = idx & 31;
#pragma unroll
            for (int x = 0; x < 4; ++x) ws[buf][kk][4 * e4 + x] = (double)wr[c][x];
        }
    };
    double acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0;
    const int nchunks = (int)((hidden + kLK - 1) / kLK);
    fetch(0);
    stash(0);
    __syncthreads();
    for (int c = 0; c < nchunks; ++c) {
        const int buf = c & 1;
        if (c + 1 < nchunks) fetch((int64_t)(c + 1) * kLK);
        const int64_t k0 = (int64_t)c * kLK;
        const int kn = (int)((hidden - k0) < kLK ? (hidden - k0) : kLK);
        for (int kk = 0; kk < kn; ++kk) {
            const double h0 = hs[buf][kk][2 * tt], h1 = hs[buf][kk][2 * tt + 1];
            double wv[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) wv[j] = ws[buf][kk][4 * te + j];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[0][j] = __builtin_fma(h0, wv[j], acc[0][j]);
                acc[1][j] = __builtin_fma(h1, wv[j], acc[1][j]);
            }
        }
        if (c + 1 < nchunks) stash(buf ^ 1);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int64_t t = t0 + 2 * tt + i;
        if (t >= tokens) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t e = e0 + 4 * te + j;
            if (e >= experts) continue;
            if (!isfinite(acc[i][j])) hm_status_or(status, HM_STATUS_NONFINITE_SCORE);
            logits[t * experts + e] = (float)acc[i][j];
        }
    }
}

// ---------------------------------------------------------------------------
// A2 logits, tiled (prefill).  Same arithmetic as router_logits_kernel: one
// sequential FP64 chain per (token, expert) in ascending k.  Workgroup tile
// 32 tokens x 64 experts, 256 threads; thread (lt, le) = (tid/16, tid%16)
// runs the 8 chains of tokens 2lt, 2lt+1 x experts 4le..4le+3, so each k
// costs three 16-byte LDS reads (two h doubles, four w doubles; the h read
// is a broadcast across the 16 threads of a token pair) for eight FMAs.
// W [32 k x 64 e] and h [32 t x 32 k] chunks come straight from global
// memory into a 4-stage LDS ring (global_load_lds) and are widened to double
// once per chunk.  Needs E % 64 == 0, H % 32 == 0 and 16-byte aligned h, w.
// ---------------------------------------------------------------------------
constexpr int kTT = 32;                // tokens per tile
constexpr int kTE = 64;                // experts per tile
constexpr int kTK = 32;                // k per chunk
constexpr int kTS = 4;                 // ring stages
constexpr int kTW = kTK * kTE * 4;     // W bytes per stage (8 KB)
constexpr int kTH = kTT * kTK * 4;     // h bytes per stage (4 KB)
constexpr int kTLPW = 3;               // 16-byte wave loads per wave per stage

__global__ __launch_bounds__(256) void router_logits_tile_kernel(
    const float* __restrict__ h, const float* __restrict__ w, int64_t tokens,
    int64_t hidden, int64_t experts, float* __restrict__ logits, int32_t* status) {
    __shared__ __attribute__((aligned(1024))) char ring[kTS][kTW + kTH];
    __shared__ __attribute__((aligned(16))) double hd[kTK][kTT];  // [k][token]
    __shared__ __attribute__((aligned(16))) double wd[kTK][kTE];  // [k][expert]
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lt = tid >> 4, le = tid & 15;
    const int64_t t0 = (int64_t)blockIdx.x * kTT;
    const int64_t e0 = (int64_t)blockIdx.y * kTE;
    // this wave's loads per stage: W rows [8w, 8w+8) as two 1 KB pieces
    // (4 rows of 64 floats each), h tokens [8w, 8w+8) x 32 k (8 lanes/token)
    const float* wsrc0 = w + (8 * wave + (lane >> 4)) * experts + e0 + 4 * (lane & 15);
    const float* wsrc1 = wsrc0 + 4 * experts;
    const int64_t tok = min(t0 + 8 * wave + (lane >> 3), tokens - 1);
    const float* hsrc = h + tok * hidden + 4 * (lane & 7);
    auto issue = [&](int slot, int64_t k0) {
        char* st = ring[slot];
        dma16(wsrc0 + k0 * experts, st + 2048 * wave);
        dma16(wsrc1 + k0 * experts, st + 2048 * wave + 1024);
        dma16(hsrc + k0, st + kTW + 1024 * wave);
    };
    double acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0;
    const int nk = (int)(hidden / kTK);
#pragma unroll
    for (int s = 0; s < kTS - 1; ++s)
        if (s < nk) issue(s, (int64_t)s * kTK);
    for (int c = 0; c < nk; ++c) {
        const int slot = c % kTS;
        if (c + kTS - 2 < nk) wait_vmcnt<(kTS - 2) * kTLPW>();
        else wait_vmcnt<0>();
        lds_barrier();  // stage c landed for every wave; chunk c-1 fully computed
        if (c + kTS - 1 < nk) issue((c + kTS - 1) % kTS, (int64_t)(c + kTS - 1) * kTK);
        {   // widen the chunk: h thread -> token tid/8, k 4*(tid%8)..+3;
            // W thread -> floats 4*tid..+3 and 1024+4*tid..+3 of [k][64]
            const float4 v = *reinterpret_cast<const float4*>(ring[slot] + kTW + 16 * tid);
            const int t = tid >> 3, kk = 4 * (tid & 7);
            hd[kk][t] = (double)v.x;
            hd[kk + 1][t] = (double)v.y;
            hd[kk + 2][t] = (double)v.z;
            hd[kk + 3][t] = (double)v.w;
            const float4 a = *reinterpret_cast<const float4*>(ring[slot] + 16 * tid);
            const float4 b = *reinterpret_cast<const float4*>(ring[slot] + 4096 + 16 * tid);
            double* w0 = &wd[0][0] + 4 * tid;
            w0[0] = (double)a.x; w0[1] = (double)a.y; w0[2] = (double)a.z; w0[3] = (double)a.w;
            w0[1024] = (double)b.x; w0[1025] = (double)b.y; w0[1026] = (double)b.z; w0[1027] = (double)b.w;
        }
        lds_barrier();
#pragma unroll
        for (int kk = 0; kk < kTK; ++kk) {
            const double2 hv = *reinterpret_cast<const double2*>(&hd[kk][2 * lt]);
            const double2 w01 = *reinterpret_cast<const double2*>(&wd[kk][4 * le]);
            const double2 w23 = *reinterpret_cast<const double2*>(&wd[kk][4 * le + 2]);
            acc[0][0] = __builtin_fma(hv.x, w01.x, acc[0][0]);
            acc[0][1] = __builtin_fma(hv.x, w01.y, acc[0][1]);
            acc[0][2] = __builtin_fma(hv.x, w23.x, acc[0][2]);
            acc[0][3] = __builtin_fma(hv.x, w23.y, acc[0][3]);
            acc[1][0] = __builtin_fma(hv.y, w01.x, acc[1][0]);
            acc[1][1] = __builtin_fma(hv.y, w01.y, acc[1][1]);
            acc[1][2] = __builtin_fma(hv.y, w23.x, acc[1][2]);
            acc[1][3] = __builtin_fma(hv.y, w23.y, acc[1][3]);
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int64_t t = t0 + 2 * lt + i;
        if (t >= tokens) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (!isfinite(acc[i][j])) hm_status_or(status, HM_STATUS_NONFINITE_SCORE);
            logits[t * experts + e0 + 4 * le + j] = (float)acc[i][j];
        }
    }
}

// ---------------------------------------------------------------------------
// A2 logits for a few tokens (decode, T <= 16), certified parallel form.
// The reference's logit is float(s_n) with s_k = fl(s_{k-1} + p_k) and
// p_k = h_k w_k (exact in double), k ascending: a chain of H dependent
// additions.  Here H is cut into kNB blocks of b = H/kNB.  Block j is summed
// sequentially from +0 (partials l_jm) beside R_j = sum_m |l_jm| and
// Q_j = sum_m |p_jm| (router_partial_kernel, one wave per block, expert
// group and token); then, per logit, the block sums are added sequentially:
// A_0 = 0, A_{j+1} = fl(A_j + B_j), S' = A_kNB, SA = sum_j |A_{j+1}|.
// Each rounding of the reference errs by at most u|s_k| (u = 2^-53), and
// |s_k| <= |A_j| + |l_jm| plus the (bounded) errors of those, so with
// R = sum R_j and P = sum Q_j
//   |s_n - S'| <= u ((b+1) SA + 2R) + u^2 (H (R + SA) + 1.01 (b^2 + H^2) P).
// Float rounding is monotone: if both ends of S' +- (that bound, inflated
// for the rounding of its own evaluation) round to the same float, it is
// the reference's logit.  Otherwise (about one logit in 10^4 - 10^5 for
// random data, and every non-finite case) the lane runs the reference's
// sequential chain.  HM_EXEC_ROUTE_SEQUENTIAL sends every logit there.
//
// R and P enter the bound only linearly, so each block stores its share
//   C_j = (2u + 2u^2 H) R_j + 2.02 u^2 (b^2 + H^2) Q_j
// and the bound is (u (b+1) + 2u^2 H) SA + sum_j C_j, inflated.
// ---------------------------------------------------------------------------
constexpr int kNB = 32;  // K blocks per logit (a multiple of 8)

__device__ __forceinline__ double block_c_term(double rs, double qs, int64_t hidden) {
    const double u = 0x1p-53;
    const double n = (double)hidden, bw = (double)(hidden / kNB);
    return (2.0 * u + 2.0 * u * u * n) * rs + 2.02 * u * u * (bw * bw + n * n) * qs;
}

// Whether the bound settles float(s_n), given the block-sum chain's result
// a, SA (sa) and the sum of the blocks' C_j (sc).
__device__ __forceinline__ bool block_sums_settle(double a, double sa, double sc,
                                                  int64_t hidden) {
    const double u = 0x1p-53;
    const double n = (double)hidden, bw = (double)(hidden / kNB);
    const double infl = 1.0 + 4.0 * n * u;  // the magnitude sums' own rounding
    const double b0 = ((u * (bw + 1.0) + 2.0 * u * u * n) * sa + sc) * infl;
    const double bc = (b0 * (1.0 + 0x1p-40) + u * fabs(a)) * (1.0 + 0x1p-50);
    const double lo = a - bc, hi = a + bc;
    return isfinite(lo) && isfinite(hi) && __float_as_uint((float)lo) == __float_as_uint((float)hi);
}

// part[t][j][e][c], c = 0, 1: B_j, C_j (block-major: a wave's 64 experts of
// one block are 1 KB in a row, written by one store and read by one load of
// the select kernel, each lane's block pair a 16-byte vector);
// grid (kNB, ceil(E/64), T), one wave, lane = expert.  The block's W rows
// (64 experts wide) go to LDS in one burst of 16-byte DMA loads
// (E % 64 == 0, b % 4 == 0, w 16-byte aligned), else per lane.
//
// With norm.gamma the kernel also is A1 RMSNorm (RMSNorm.cpp:65-77; the
// transformer block runs it on the router's input, TransformerBlock.cpp:
// 88-104): every wave of a token forms the row's tree sum of squares,
// brackets the reference's sequential sum by it as rmsnorm_kernel does, and
// normalises the elements of its own K block; an element the bracket does
// not settle makes the wave take the sequential sum itself, which gives the
// reference's value for every element.  The waves of expert group 0 write
// their blocks to norm.x_out.
constexpr int kPK = 64;  // k per LDS chunk of a block

__global__ __launch_bounds__(64) void router_partial_kernel(
    const float* __restrict__ h, const float* __restrict__ w, int hidden, int experts,
    double* __restrict__ part, int32_t* __restrict__ zero_ctr, int n_zero, hm_norm_fold norm) {
    extern __shared__ float s_row[];  // with the norm: the row (hidden floats)
    __shared__ double s_h[kPK];                                        // broadcast reads
    __shared__ __attribute__((aligned(1024))) float s_w[kPK][HM_WAVE];  // [k][lane]
    const int lane = threadIdx.x;
    // completion counters of the later kernels of a fused decode step start
    // at zero (they run after this kernel has finished)
    if (zero_ctr && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0)
        for (int i = lane; i < n_zero; i += HM_WAVE) zero_ctr[i] = 0;
    const int j = blockIdx.x, t = blockIdx.z;
    const int e0 = blockIdx.y * HM_WAVE;
    const int e = e0 + lane;
    const bool live = e < experts;
    const int b = hidden / kNB;
    const bool full = experts % HM_WAVE == 0 && b % 4 == 0 && (uintptr_t)w % 16 == 0;
    const int k0 = j * b;
    const float* hrow = h + (int64_t)t * hidden;
    const float* hp = hrow + k0;
    const bool fold = norm.gamma != nullptr;
    // the whole row in one burst of 16-byte loads (at most 16 per lane)
    const bool row4 = hidden % 256 == 0 && hidden <= 16 * 256 && (uintptr_t)h % 16 == 0;
    double inv_lo = 0.0, inv_hi = 0.0, inv_seq = 0.0;
    bool have_seq = false;
    float4 v[16];  // the row (row4): kept for an LDS copy if the sequential sum is needed
    double acc = 0.0, rs = 0.0, qs = 0.0;
    for (int c0 = 0; c0 < b; c0 += kPK) {
        const int kc = min(kPK, b - c0);
        __builtin_amdgcn_wave_barrier();
        // unconditional loads from clamped addresses (a load under a branch
        // is waited for at the branch's end), masked once they are in
        const int lc = min(lane, kc - 1);
        float hv = hp[c0 + lc];
        const float gv = (fold ? norm.gamma + k0 : hp)[c0 + lc];
        if (full) {
            // lane l: row 4i + l/16, floats 4*(l%16) .. +3 of the 64-expert row
            const float* src = w + (int64_t)(k0 + c0 + (lane >> 4)) * experts + e0 + 4 * (lane & 15);
            for (int i = 0; i < kc / 4; ++i) dma16(src + (int64_t)4 * i * experts, &s_w[4 * i][0]);
        }
        if (fold) {
            if (c0 == 0) {
                // the row's squares, in any order (their loads overlap the
                // block's W burst)
                double ss = 0.0;
                if (row4) {
                    const float4* r4 = reinterpret_cast<const float4*>(hrow);
                    const int n4 = hidden >> 8;
#pragma unroll
                    for (int i = 0; i < 16; ++i) v[i] = r4[lane + HM_WAVE * min(i, n4 - 1)];
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const double q = ((double)v[i].x * v[i].x + (double)v[i].y * v[i].y) +
                                         ((double)v[i].z * v[i].z + (double)v[i].w * v[i].w);
                        ss += i < n4 ? q : 0.0;
                    }
                } else {
                    for (int i = lane; i < hidden; i += HM_WAVE) {
                        const float v = hrow[i];
                        ss += (double)v * v;
                        s_row[i] = v;
                    }
                }
                const double s_fast = hm_wave_sum_f64(ss);
                const double d = hm_rms_sum_slack(hidden);
                inv_lo = hm_inv_rms(s_fast * (1.0 + d), (double)hidden, (double)norm.eps);
                inv_hi = hm_inv_rms(s_fast * (1.0 - d), (double)hidden, (double)norm.eps);
            }
            hv = lane < kc ? hv : 0.0f;
            const double g = lane < kc ? (double)gv : 0.0;
            const float a = (float)((double)hv * inv_lo * g);
            const float bb = (float)((double)hv * inv_hi * g);
            if (!have_seq && (norm.force_seq || __any(__float_as_uint(a) != __float_as_uint(bb)))) {
                // the sequential sum over the row's LDS copy (every lane
                // the same, broadcast reads)
                if (row4) {
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (i < (hidden >> 8)) reinterpret_cast<float4*>(s_row)[lane + HM_WAVE * i] = v[i];
                }
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                inv_seq = hm_inv_rms(hm_rms_sum_seq(s_row, hidden), (double)hidden, (double)norm.eps);
                have_seq = true;
            }
            hv = have_seq ? (float)((double)hv * inv_seq * g) : a;
            if (blockIdx.y == 0 && lane < kc) norm.x_out[(int64_t)t * hidden + k0 + c0 + lane] = hv;
        }
        s_h[lane] = lane < kc ? (double)hv : 0.0;
        if (full) {
            wait_vmcnt<0>();
        } else {
            for (int i = 0; i < kc; ++i) s_w[i][lane] = live ? w[(int64_t)(k0 + c0 + i) * experts + e] : 0.0f;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        auto step = [&](double hk, double wd) __attribute__((always_inline)) {
            acc = __builtin_fma(hk, wd, acc);  // == acc + hk * wd (the product is exact)
            rs += fabs(acc);
            qs = __builtin_fma(fabs(hk), fabs(wd), qs);
        };
        if (kc == kPK) {
            // a whole chunk: the LDS values of the next kRSub steps are read
            // while the current ones are chained, so the chain does not wait
            // for an LDS read every other step (same steps, same order)
            constexpr int kRSub = 16;
            double hb[2][kRSub];
            float wb[2][kRSub];
            auto fetch = [&](int buf, int i0) __attribute__((always_inline)) {
#pragma unroll
                for (int i = 0; i < kRSub; ++i) {
                    hb[buf][i] = s_h[i0 + i];
                    wb[buf][i] = s_w[i0 + i][lane];
                }
            };
            fetch(0, 0);
#pragma unroll
            for (int c = 0; c < kPK / kRSub; ++c) {
                if (c + 1 < kPK / kRSub) fetch((c + 1) & 1, (c + 1) * kRSub);
#pragma unroll
                for (int i = 0; i < kRSub; ++i) step(hb[c & 1][i], (double)wb[c & 1][i]);
            }
        } else {
            for (int i = 0; i < kc; ++i) step(s_h[i], (double)s_w[i][lane]);
        }
    }
    if (live) {
        double2* o = reinterpret_cast<double2*>(part + (((int64_t)t * kNB + j) * experts + e) * 2);
        *o = make_double2(acc, block_c_term(rs, qs, hidden));
    }
}

// One logit from its block partials (see above); *settled is false when
// the bound does not settle the float (the caller then runs the sequential
// chain).  pp: this logit's B_0, C_0 (part + (t*kNB*E + e) * 2); block j's
// pair sits 2 E doubles further on per block.
__device__ __forceinline__ float block_logit(const double* __restrict__ pp, int64_t experts,
                                             int64_t hidden, bool force_seq, bool* settled) {
    // all 64 values in 32 vector loads (each block's B_j and C_j in one,
    // so that both sums need every load), then the dependent chain
    typedef int hm_i4 __attribute__((ext_vector_type(4)));
    hm_i4 raw[kNB];
#pragma unroll
    for (int i = 0; i < kNB; ++i) raw[i] = *reinterpret_cast<const hm_i4*>(pp + (int64_t)i * 2 * experts);
    // (every load goes out before the first is used: otherwise the compiler
    // splits each pair and issues the C halves only after the B chain)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < kNB; ++i) asm volatile("" : "+v"(raw[i]));
    double a = 0.0, sa = 0.0, sc = 0.0;
#pragma unroll
    for (int i = 0; i < kNB; ++i) {
        const double2 bc = __builtin_bit_cast(double2, raw[i]);
        a += bc.x;
        sa += fabs(a);
        sc += bc.y;
    }
    *settled = !force_seq && block_sums_settle(a, sa, sc, hidden);
    return (float)a;
}

// The reference's sequential chain s_k = fl(s_{k-1} + h_k w_k) (the
// product is exact in double, so fl(s + p) = fma(h, w, s)) for the logit of
// expert e0 + lane of every lane whose bit is set in `need`, one logit at a time:
// the whole wave forms 64 exact products at once into LDS (prod: 64
// doubles of this wave) and the owning lane adds them in order, 16 reads
// ahead of its additions.  hidden % 16 == 0.  Returns the owning lane's
// float logit (others: v unchanged).
__device__ __forceinline__ float chain_logits(unsigned long long need, int lane, float v, int64_t e0,
                                              const float* __restrict__ hrow,
                                              const float* __restrict__ w, int64_t hidden,
                                              int64_t experts, double* prod, int32_t* status) {
    while (need) {
        const int owner = __ffsll((long long)need) - 1;
        need &= need - 1;
        const int64_t eo = e0 + owner;
        double acc = 0.0;
        for (int64_t c0 = 0; c0 < hidden; c0 += HM_WAVE) {
            const int64_t k = min(c0 + lane, hidden - 1);
            const double p = (double)hrow[k] * (double)w[k * experts + eo];
            __builtin_amdgcn_wave_barrier();
            prod[lane] = p;
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            if (lane == owner) {
                const int n = (int)min((int64_t)HM_WAVE, hidden - c0);
                for (int i = 0; i < n; i += 16) {
                    double r[16];
#pragma unroll
                    for (int u = 0; u < 16; ++u) r[u] = prod[i + u];
#pragma unroll
                    for (int u = 0; u < 16; ++u) acc += r[u];
                }
            }
        }
        if (lane == owner) {
            if (!isfinite(acc)) hm_status_or(status, HM_STATUS_NONFINITE_SCORE);
            v = (float)acc;
        }
    }
    return v;
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
// Writes ids/scores [t, r] in rank order.
// ---------------------------------------------------------------------------
// Softmax, top-k and renormalisation of one token's logits v (one wave; lane
// holds experts lane + 64 j); writes ids/scores [t, r] in rank order.
// A token whose selection failed (the status word says so): placeholder ids
// 0..top_k-1 with zero scores, so that the permutation and expert stages that
// follow on the stream stay in range.
// A token's id and score stores; `coherent`: device-scope stores (sc1,
// written through to the device's coherence point), for a workgroup of
// another XCD that reads them once this one has arrived at the completion
// counter (no L2 write-back needed).
template <typename V>
__device__ __forceinline__ void hm_store_pair(V* p, V v, bool coherent) {
    if (coherent) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else *p = v;
}
template <typename V>
__device__ __forceinline__ V hm_load_pair(const V* p, bool coherent) {
    return coherent ? __hip_atomic_load(const_cast<V*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                    : *p;
}

__device__ __forceinline__ void select_failed(int lane, int64_t t, int32_t top_k,
                                              uint32_t* __restrict__ ids,
                                              float* __restrict__ scores,
                                              uint32_t* l_ids = nullptr,
                                              float* l_scores = nullptr, bool coherent = false) {
    if (lane < top_k) {
        hm_store_pair(&ids[t * top_k + lane], (uint32_t)lane, coherent);
        hm_store_pair(&scores[t * top_k + lane], 0.0f, coherent);
        if (l_ids) {
            l_ids[lane] = (uint32_t)lane;
            l_scores[lane] = 0.0f;
        }
    }
}

template <int EPL>
__device__ __forceinline__ void select_token(float (&v)[EPL], const bool (&valid)[EPL], int lane,
                                             int wave, int64_t t, int64_t experts, int32_t top_k,
                                             uint32_t flags, uint32_t* __restrict__ ids,
                                             float* __restrict__ scores, int32_t* status,
                                             float* seq_lds, uint32_t* l_ids = nullptr,
                                             float* l_scores = nullptr, bool coherent = false) {
    // (l_ids, l_scores: optional LDS copies of this token's ids and scores;
    // coherent: device-scope stores, hm_store_pair)
    if (flags & HM_ROUTE_SOFTMAX) {
        float m = -__uint_as_float(0x7f800000u);
#pragma unroll
        for (int j = 0; j < EPL; ++j) if (valid[j]) m = fmaxf(m, v[j]);
        m = hm_wave_max_dpp(m);
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
            den = hm_wave_sum_f64_dpp(part);
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
            select_failed(lane, t, top_k, ids, scores, l_ids, l_scores, coherent);
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
    // k rounds of the wave maximum (keys are unique: the winner's own key
    // is the one that equals it); lane r keeps the r-th id, and after the
    // rounds fetches its score from the lane that holds it
    uint32_t my_id = 0;
    for (int r = 0; r < top_k; ++r) {
        unsigned long long best = 0ull;
#pragma unroll
        for (int j = 0; j < EPL; ++j) best = key[j] > best ? key[j] : best;
        best = hm_wave_max_u64_bcast(best);
#pragma unroll
        for (int j = 0; j < EPL; ++j) key[j] = key[j] == best ? 0ull : key[j];
        if (lane == r) my_id = 0xffffffffu - (uint32_t)(best & 0xffffffffull);
    }
    float my_score = 0.0f;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        const float c = __shfl(v[j], (int)(my_id % HM_WAVE), HM_WAVE);
        if ((int)(my_id / HM_WAVE) == j) my_score = c;
    }
    double sel_sum = 0.0;  // rank order, uniform across lanes
    for (int r = 0; r < top_k; ++r)
        sel_sum += (double)__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_score), r));
    if (flags & HM_ROUTE_RENORM) {
        if (!(isfinite(sel_sum) && sel_sum != 0.0)) {
            if (lane == 0) hm_status_or(status, HM_STATUS_RENORM_FAILED);
            select_failed(lane, t, top_k, ids, scores, l_ids, l_scores, coherent);
            return;
        }
        my_score = (float)((double)my_score / sel_sum);
    }
    if (lane < top_k) {
        hm_store_pair(&ids[t * top_k + lane], my_id, coherent);
        hm_store_pair(&scores[t * top_k + lane], my_score, coherent);
        if (l_ids) {
            l_ids[lane] = my_id;
            l_scores[lane] = my_score;
        }
    }
}

template <int EPL>
__global__ __launch_bounds__(kBlock) void router_select_kernel(
    const float* __restrict__ logits, int64_t tokens, int64_t experts,
    int32_t top_k, uint32_t flags, uint32_t* __restrict__ ids,
    float* __restrict__ scores, int32_t* status) {
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
    select_token<EPL>(v, valid, lane, wave, t, experts, top_k, flags, ids, scores, status, seq_lds);
}

// The stable counting sort of permute_count/scatter for at most
// kSmallPairs pairs, by one workgroup (NT threads): counts and offsets
// from an LDS histogram and a block scan, each pair's rank among the
// earlier pairs of its expert by a scan of the ids in LDS.  Ids past the
// expert count (left behind by a routing failure the status word reports)
// are treated as the last expert so that every position stays in range.
constexpr int kSmallPairs = 1024;

template <int NT>
__device__ void permute_small(const uint32_t* __restrict__ ids, const float* __restrict__ scores,
                              int pairs, int top_k, int experts, int32_t* __restrict__ counts,
                              int32_t* __restrict__ offsets, int32_t* __restrict__ perm_tokens,
                              float* __restrict__ perm_weights, int32_t* __restrict__ slots,
                              bool coherent = false) {
    // (coherent: ids and scores read device-scope, hm_load_pair)
    constexpr int EPT = 1024 / NT;  // experts per thread in the scan (E <= 1024)
    __shared__ int s_cnt[1024];
    __shared__ int s_off[1024];
    __shared__ int s_ids[kSmallPairs];
    __shared__ int s_wsum[NT / HM_WAVE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < experts; i += NT) s_cnt[i] = 0;
    __syncthreads();
    for (int p = tid; p < pairs; p += NT) {
        const uint32_t e = hm_load_pair(&ids[p], coherent);
        const int ec = e < (uint32_t)experts ? (int)e : experts - 1;
        s_ids[p] = ec;
        atomicAdd(&s_cnt[ec], 1);
    }
    __syncthreads();
    // exclusive scan over experts: thread tid owns experts EPT*tid .. +EPT-1
    int v[EPT], tot = 0;
#pragma unroll
    for (int q = 0; q < EPT; ++q) {
        const int e = EPT * tid + q;
        v[q] = e < experts ? s_cnt[e] : 0;
        tot += v[q];
    }
    int incl = tot;
#pragma unroll
    for (int sft = 1; sft < 64; sft <<= 1) {
        const int o = __shfl_up(incl, sft, 64);
        if (lane >= sft) incl += o;
    }
    if (lane == 63) s_wsum[wave] = incl;
    __syncthreads();
    int base = incl - tot;
    for (int wv = 0; wv < wave; ++wv) base += s_wsum[wv];
#pragma unroll
    for (int q = 0; q < EPT; ++q) {
        const int e = EPT * tid + q;
        if (e < experts) {
            s_off[e] = base;
            counts[e] = v[q];
            offsets[e] = base;
            if (e == experts - 1) offsets[experts] = base + v[q];
        }
        base += v[q];
    }
    __syncthreads();
    for (int p = tid; p < pairs; p += NT) {
        const int e = s_ids[p];
        int rank = 0;
        for (int q = 0; q < p; ++q) rank += s_ids[q] == e;
        const int pos = s_off[e] + rank;
        perm_tokens[pos] = p / top_k;
        perm_weights[pos] = hm_load_pair(&scores[p], coherent);
        slots[p] = pos;
    }
}

// The grouping of permute_small for P <= 64 pairs by one wave, in
// registers: lane p holds pair p (its id, clamped to the expert count as
// permute_small does, and score); its position is the number of pairs with
// a smaller expert plus the earlier pairs of its own expert (the stable
// counting sort), the lanes' experts lane + 64 j count their pairs and
// those of smaller experts (counts, offsets), each pair's id read in turn
// across the wave.
template <int EPL>
__device__ __forceinline__ void permute_wave(uint32_t id, float score, int pairs, int top_k,
                                             int experts, int32_t* __restrict__ counts,
                                             int32_t* __restrict__ offsets,
                                             int32_t* __restrict__ perm_tokens,
                                             float* __restrict__ perm_weights,
                                             int32_t* __restrict__ slots) {
    const int lane = threadIdx.x & (HM_WAVE - 1);
    const int ep = lane < pairs ? (int)min(id, (uint32_t)(experts - 1)) : INT_MAX;
    int less = 0, same = 0;
    int cnt[EPL], off[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) cnt[j] = off[j] = 0;
    for (int q = 0; q < pairs; ++q) {
        const int eq = __builtin_amdgcn_readlane(ep, q);
        less += eq < ep;
        same += (eq == ep) & (q < lane);
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const int e = lane + HM_WAVE * j;
            cnt[j] += eq == e;
            off[j] += eq < e;
        }
    }
    if (lane < pairs) {
        const int pos = less + same;
        perm_tokens[pos] = lane / top_k;
        perm_weights[pos] = score;
        slots[lane] = pos;
    }
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        const int e = lane + HM_WAVE * j;
        if (e < experts) {
            counts[e] = cnt[j];
            offsets[e] = off[j];
            if (e == experts - 1) offsets[experts] = off[j] + cnt[j];
        }
    }
}

// Select over logits formed from the decode partials (and written to
// `logits` too).  !SPLIT: NW tokens per workgroup, one per wave.  SPLIT: one
// token per workgroup, its rows of 64 logits shared out over the NW waves
// so that all their loads are in flight together (each token reads 2 kNB
// doubles per logit, 64 KB at E = 128, that other CUs wrote), wave 0
// selecting.  With PERMUTE the workgroup that finishes last (a device
// counter, zeroed by router_partial_kernel) also sorts the pairs into
// expert groups, which is hm_permute's result: one launch fewer per decode
// step; a single workgroup hands its ids and scores over in LDS.
template <int EPL, bool PERMUTE, int NW, bool SPLIT>
__global__ __launch_bounds__(NW * HM_WAVE) void router_select_partial_kernel(
    const float* __restrict__ h, const float* __restrict__ w, const double* __restrict__ part,
    int64_t tokens, int64_t hidden, int64_t experts, int32_t top_k, uint32_t flags,
    float* __restrict__ logits, uint32_t* __restrict__ ids, float* __restrict__ scores,
    int32_t* status, int32_t* __restrict__ done_ctr, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ perm_tokens,
    float* __restrict__ perm_weights, int32_t* __restrict__ slots, hm_row_quant xq) {
    extern __shared__ float seq_lds[];  // NW * experts floats
    __shared__ double s_prod[NW][HM_WAVE];
    // one workgroup: the grouping reads the ids and scores from LDS copies
    __shared__ uint32_t s_sel_ids[PERMUTE ? NW * 64 : 1];
    __shared__ float s_sel_sc[PERMUTE ? NW * 64 : 1];
    // SPLIT: the token's logits, rows of 64 experts shared out over the waves
    __shared__ float s_lg[SPLIT ? EPL : 1][HM_WAVE];
    const bool local = PERMUTE && gridDim.x == 1;
    // several workgroups: the last to arrive groups every token's pairs, so
    // the ids and scores go out device-coherent
    const bool shared = PERMUTE && gridDim.x > 1;
    const int lane = threadIdx.x & (HM_WAVE - 1);
    const int wave = threadIdx.x / HM_WAVE;
    const bool force_seq = (flags & HM_EXEC_ROUTE_SEQUENTIAL) != 0;
    // one logit row j (experts 64 j + lane) of token t: its block sums, and
    // the reference's chain where the bound leaves it open
    auto logit_row = [&](int64_t t, int j, bool& valid) __attribute__((always_inline)) -> float {
        const int64_t e = lane + (int64_t)HM_WAVE * j;
        valid = e < experts;
        bool settled;
        // (lanes past the experts read the last expert's: no branch around the loads)
        float v = block_logit(part + (t * kNB * experts + (valid ? e : experts - 1)) * 2, experts,
                              hidden, force_seq, &settled);
        if (!valid) {
            v = 0.0f;
            settled = true;
        }
        v = chain_logits(__ballot(valid && !settled), lane, v, (int64_t)HM_WAVE * j,
                         h + t * hidden, w, hidden, experts, s_prod[wave], status);
        if (valid) logits[t * experts + e] = v;
        return v;
    };
    if constexpr (SPLIT) {
        // one token per workgroup: wave w forms rows w, w + NW, .., so that
        // every row's loads are in flight at once; wave 0 selects
        const int64_t t = blockIdx.x;
        for (int j = wave; j < EPL; j += NW) {
            bool valid;
            s_lg[j][lane] = logit_row(t, j, valid);
        }
        __syncthreads();
        if (wave == 0) {
            float v[EPL];
            bool valid[EPL];
#pragma unroll
            for (int j = 0; j < EPL; ++j) {
                v[j] = s_lg[j][lane];
                valid[j] = lane + (int64_t)HM_WAVE * j < experts;
            }
            select_token<EPL>(v, valid, lane, 0, t, experts, top_k, flags, ids, scores, status,
                              seq_lds, local ? s_sel_ids : nullptr, local ? s_sel_sc : nullptr,
                              shared);
            if (local && top_k <= HM_WAVE) {
                // one token: its grouping by this wave, from the LDS copies
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                const int ln = lane < top_k ? lane : 0;
                permute_wave<EPL>(s_sel_ids[ln], s_sel_sc[ln], top_k, top_k, (int)experts,
                                  counts, offsets, perm_tokens, perm_weights, slots);
            }
        }
        // the token's row in fixed-point digits for the INT8 expert GEMMs,
        // by the last wave (beside wave 0's selection when there are two)
        if (xq.digits && wave == NW - 1) {
            const int nv = (int)(hidden / 256);
            const hm_dlay lay = hm_dlay_x(xq.limbs, hidden);
            int8_t* d = xq.digits + t * lay.row;
            int32_t* ds = xq.dsum ? xq.dsum + t : nullptr;
            switch (xq.limbs) {
            case 1: hm_quantize_row_wave<1>(h + t * hidden, nv, d, lay, xq.scales + t, ds, tokens); break;
            case 2: hm_quantize_row_wave<2>(h + t * hidden, nv, d, lay, xq.scales + t, ds, tokens); break;
            default: hm_quantize_row_wave<3>(h + t * hidden, nv, d, lay, xq.scales + t, ds, tokens); break;
            }
        }
        if (local && top_k <= HM_WAVE) return;
    } else {
        // one token per wave
        const int64_t t = (int64_t)blockIdx.x * NW + wave;
        if (t < tokens) {
            float v[EPL];
            bool valid[EPL];
#pragma unroll
            for (int j = 0; j < EPL; ++j) v[j] = logit_row(t, j, valid[j]);
            select_token<EPL>(v, valid, lane, wave, t, experts, top_k, flags, ids, scores, status,
                              seq_lds, local ? s_sel_ids + wave * top_k : nullptr,
                              local ? s_sel_sc + wave * top_k : nullptr, shared);
        }
    }
    if constexpr (PERMUTE) {
        if (gridDim.x > 1) {
            // Arrival without a write-back of this XCD's L2: the ids and
            // scores were stored device-coherent (sc1); once this wave's
            // stores are complete (vmcnt 0, every wave) the workgroup counts
            // in, and the last one reads them device-coherent too.
            __shared__ int s_last;
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (threadIdx.x == 0)
                s_last = __hip_atomic_fetch_add(done_ctr, 1, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT) == (int)gridDim.x - 1;
            __syncthreads();
            if (!s_last) return;
        } else {
            __syncthreads();  // one workgroup: its own ids and scores
        }
        permute_small<NW * HM_WAVE>(local ? s_sel_ids : ids, local ? s_sel_sc : scores,
                                    (int)(tokens * top_k), top_k, (int)experts, counts, offsets,
                                    perm_tokens, perm_weights, slots, shared);
    }
}

// ---------------------------------------------------------------------------
// One-token decode step: router_select_partial_kernel's select, redone by
// every workgroup of the gate/up slice launch, then that workgroup's slice
// (hm_gemv_slice.h).  One token's select reads 2 kNB doubles per logit
// (32 KB at E = 128) that every XCD's L2 serves to its workgroups, and
// costs a few hundred cycles of FP64 arithmetic: less than the launch it
// replaces.  Workgroup (bx, by): columns 8 bx .. +7 of the by-th selected
// expert in ascending id (its grouped row is by: one token, distinct
// experts).  Workgroup (0, 0) also writes the routing results (logits, ids,
// scores, the groups, the status word) for the down kernel and the caller;
// the others keep theirs in LDS.  Same results as the two kernels it
// replaces: the same functions on the same partials.
// ---------------------------------------------------------------------------
// Workgroup phases: (1) the token row's loads, then every wave loads a
// quarter (E <= 64: an eighth) of one logit row's block partials, all in
// flight at once, and puts the blocks' B_j and its share of sum C_j in LDS;
// (2) wave j forms row j's block-sum chain and bound from LDS (as
// block_logit; the C_j summed in another order, which the bound's
// inflation covers), the reference's chain where the bound leaves a logit
// open; (3) wave 0: softmax, top-k, renormalisation (select_token), the lead
// workgroup writes the results and the groups; (4) the slice.
template <int EPL, int LJ>
__global__ __launch_bounds__(kGvThreads) void select_gateup_kernel(
    const float* __restrict__ h, const float* __restrict__ w, const double* __restrict__ part,
    int64_t hidden, int64_t experts, int32_t top_k, uint32_t flags, float* __restrict__ logits,
    uint32_t* __restrict__ ids, float* __restrict__ scores, int32_t* status,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ perm_tokens, float* __restrict__ perm_weights,
    int32_t* __restrict__ slots, int64_t inter, const int8_t* __restrict__ packed,
    const float* __restrict__ scale, const int32_t* __restrict__ zp, float* __restrict__ z) {
    static_assert(EPL == 1 || EPL == 2, "at most two rows of 64 logits (LDS)");
    constexpr int WPR = kGvWaves / EPL;  // waves per logit row
    constexpr int BPW = kNB / WPR;       // blocks per wave
    typedef int hm_i4 __attribute__((ext_vector_type(4)));
    extern __shared__ __attribute__((aligned(16))) float s_x[];  // the token row (K32 floats)
    __shared__ double s_b[EPL][kNB][HM_WAVE];
    __shared__ double s_c[EPL][WPR][HM_WAVE];
    __shared__ double s_prod[EPL][HM_WAVE];
    __shared__ float s_seq[EPL * HM_WAVE];
    __shared__ float s_lg[EPL][HM_WAVE];
    __shared__ uint32_t s_sel_ids[HM_WAVE], s_own_ids[HM_WAVE];
    __shared__ float s_sel_sc[HM_WAVE], s_own_sc[HM_WAVE];
    const int tid = threadIdx.x, lane = tid & (HM_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool lead = blockIdx.x == 0 && blockIdx.y == 0;
    int32_t* st = lead ? status : nullptr;
    // (1) the token row (K = hidden, a multiple of 32: no padding), then the
    // partials of row j, blocks q BPW .. +BPW-1
    const int k4 = (int)(hidden / 4);
    float4 xa[2];
#pragma unroll
    for (int u = 0; u < 2; ++u)
        xa[u] = reinterpret_cast<const float4*>(h)[min(tid + u * kGvThreads, k4 - 1)];
    {
        const int j = wave / WPR, q = wave % WPR;
        const int64_t e = lane + (int64_t)HM_WAVE * j;
        const double* pp = part + (e < experts ? e : experts - 1) * 2 +
                           (int64_t)q * BPW * 2 * experts;
        hm_i4 raw[BPW];
#pragma unroll
        for (int i = 0; i < BPW; ++i) raw[i] = *reinterpret_cast<const hm_i4*>(pp + (int64_t)i * 2 * experts);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < BPW; ++i) asm volatile("" : "+v"(raw[i]));
#pragma unroll
        for (int u = 0; u < 2; ++u)
            if (tid + u * kGvThreads < k4) reinterpret_cast<float4*>(s_x)[tid + u * kGvThreads] = xa[u];
        double cs = 0.0;
#pragma unroll
        for (int i = 0; i < BPW; ++i) {
            const double2 bc = __builtin_bit_cast(double2, raw[i]);
            s_b[j][q * BPW + i][lane] = bc.x;
            cs += bc.y;
        }
        s_c[j][q][lane] = cs;
    }
    __syncthreads();
    // (2) the logits, row j by wave j
    if (wave < EPL) {
        const int64_t e = lane + (int64_t)HM_WAVE * wave;
        const bool valid = e < experts;
        double a = 0.0, sa = 0.0, sc = 0.0;
#pragma unroll
        for (int i = 0; i < kNB; ++i) {
            a += s_b[wave][i][lane];
            sa += fabs(a);
        }
#pragma unroll
        for (int q = 0; q < WPR; ++q) sc += s_c[wave][q][lane];
        const bool settled = !valid || ((flags & HM_EXEC_ROUTE_SEQUENTIAL) == 0 &&
                                        block_sums_settle(a, sa, sc, hidden));
        float v = valid ? (float)a : 0.0f;
        v = chain_logits(__ballot(valid && !settled), lane, v, (int64_t)HM_WAVE * wave, h, w,
                         hidden, experts, s_prod[wave], st);
        if (lead && valid) logits[e] = v;
        s_lg[wave][lane] = v;
    }
    __syncthreads();
    // (3) softmax, top-k, renormalisation (wave 0); the lead workgroup
    // writes the results and the groups
    if (wave == 0) {
        float v[EPL];
        bool valid[EPL];
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            v[j] = s_lg[j][lane];
            valid[j] = lane + (int64_t)HM_WAVE * j < experts;
        }
        select_token<EPL>(v, valid, lane, 0, 0, experts, top_k, flags, lead ? ids : s_own_ids,
                          lead ? scores : s_own_sc, st, s_seq, s_sel_ids, s_sel_sc);
        if (lead) {
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            const int ln = lane < top_k ? lane : 0;
            permute_wave<EPL>(s_sel_ids[ln], s_sel_sc[ln], top_k, top_k, (int)experts, counts,
                              offsets, perm_tokens, perm_weights, slots);
        }
    }
    __syncthreads();
    // (4) this workgroup's expert: the selected id of rank by (ids clamped to
    // the expert count, as the grouping does), and its slice
    const uint32_t my = lane < top_k ? min(s_sel_ids[lane], (uint32_t)(experts - 1)) : 0xffffffffu;
    int rank = 0;
    for (int q = 0; q < top_k; ++q) rank += (uint32_t)__shfl((int)my, q, HM_WAVE) < my;
    const unsigned long long hit = __ballot(lane < top_k && rank == (int)blockIdx.y);
    const int e = hit ? __builtin_amdgcn_readlane((int)my, __ffsll((long long)hit) - 1) : -1;
    gateup_slice_body<1, LJ, true, 1>(blockIdx.x, blockIdx.y,
                                      hm_slice_pre{e, (int)blockIdx.y, 1, 0}, h, nullptr, hidden,
                                      inter, experts, packed, scale, zp, nullptr, 1, z);
}

// ---------------------------------------------------------------------------
// A2 logits for prefill batches on the FP64 matrix cores, certified.
//
// router_mfma_kernel sums the exact products p_k = h_k w_k (double) with
// v_mfma_f64_16x16x4_f64 in an order of its own: K is cut into `splits`
// ranges (one per workgroup layer of the grid) and each range into chunks
// of 16, of which MFMA step j takes k = 4g + j for the four k-slots g; the
// kernel also returns the norms of h's rows and W's columns per
// range.  router_select_split_kernel adds the S ranges' partials P'_r in
// order (S'_r after range r, S' = S'_{S-1}) and bounds |S' - s_n| from
// these, with m = n / S terms per range, A_r = sum_{k in r} |p_k| <=
// ||h_r|| ||w_e,r|| (Cauchy-Schwarz per range) and u = 2^-53:
//   - each range partial: any summation tree of m terms errs by at most
//     gamma_m A_r, doubled to cover an internal rounding mode of the
//     matrix cores of up to 2u (g2 = 2mu / (1 - 2mu));
//   - the additions of the partials: u |S'_r| each; with the above
//     D = g2 sum_r A_r + u sum_r |S'_r| bounds |S' - S_n| and every prefix
//     |S'_{r-1} - S_{rm}| (S_k: the exact partial sums);
//   - the reference's chain: its step k errs by at most u' |s_k| (u' =
//     u / (1 - u)), |s_k| <= |S_k| + B and, for k in range r, |S_k| <=
//     |S'_{r-1}| + D + A_r, so B <= u' m (sum_r |S'_{r-1}| + S D + sum_r
//     A_r) / (1 - n u');
// the bound is B + D, inflated by 2^-20 for the norms' and the bound's own
// rounding (relative errors below 2^-40 here).  float(S') is kept when both
// ends of S' +- bound round to the same float; otherwise (about 0.05 % of
// the logits for N(0,1) rows and N(0, 0.02) weights at H = 2048 in four
// ranges, and every non-finite case) the logit takes the fallbacks below.
//
// Workgroup: 4 waves x 16 tokens, 64 experts as 4 interleaved MFMA chains
// (chain q holds experts e0 + 4n + q, n = 0..15), so that each W load is a
// float4 of 4 consecutive experts (one per chain) and each h load a float4
// of 4 consecutive k (one per MFMA step).  Lane (g, i) = (lane/16, lane%16)
// supplies A = h[t0 + i][k] and B = W[k][e0 + 4i + q]; its result register
// r holds D[g + 4r][i] = the logit of token t0 + g + 4r, expert e0 + 4i + q.
// Needs E % 64 == 0, H % (16 * splits) == 0, 16-byte aligned h and w.
// ---------------------------------------------------------------------------
constexpr int kMT = 64;   // tokens per workgroup
constexpr int kME = 64;   // experts per workgroup
constexpr int kMaxSplits = 8;
constexpr int kMS = 4;    // LDS ring stages of one 16-k chunk each
constexpr int kMW = 4096; // W bytes per stage: [16 k][64 e] floats
constexpr int kMH = 4096; // h bytes per stage: [64 t][16 k] floats
typedef double hm_double4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void router_mfma_kernel(
    const float* __restrict__ h, const float* __restrict__ w, int tokens, int hidden,
    int experts, int ksplit, double* __restrict__ part, float* __restrict__ wt,
    double* __restrict__ hnorm_r, double* __restrict__ wnorm_r, int32_t* __restrict__ hist, int hist_n) {
    __shared__ __attribute__((aligned(1024))) char ring[kMS][kMW + kMH];
    // the permutation's chunk histograms, counted by the select kernel
    for (int i = blockIdx.x * 256 + threadIdx.x; i < hist_n; i += gridDim.x * 256) hist[i] = 0;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, i = lane & 15;
    const int eblocks = experts / kME;
    const int tblocks = (tokens + kMT - 1) / kMT;
    const int eb = blockIdx.x % eblocks;
    const int tb = (blockIdx.x / eblocks) % tblocks;
    const int sp = blockIdx.x / (eblocks * tblocks);
    const int t0 = tb * kMT + 16 * wave;
    const int e0 = eb * kME;
    const int tok = t0 + i;
    const bool live = tok < tokens;
    const int kb = sp * ksplit;
    const int nk = ksplit / 16;
    // Each wave stages a quarter of a chunk: W rows 4*wave .. +3 (1 KB, lane
    // l: row 4*wave + l/16, experts 4*(l%16) .. +3) and its own 16 tokens' h
    // (1 KB, lane l: token 16*wave + l/4, k 4*(l%4) .. +3); rows of tokens
    // past the end repeat the last token and are masked below.
    const float* wsrc = w + (int64_t)(kb + 4 * wave + (lane >> 4)) * experts + e0 + 4 * (lane & 15);
    const int htok = min(t0 + (lane >> 2), tokens - 1);
    const float* hsrc = h + (int64_t)htok * hidden + kb + 4 * (lane & 3);
    auto issue = [&](int slot, int c) {
        dma16(wsrc + (int64_t)16 * c * experts, ring[slot] + 1024 * wave);
        dma16(hsrc + 16 * c, ring[slot] + kMW + 1024 * wave);
    };
    const bool wnorm = tb == 0 && wave == 0;  // one wave per (range, expert block)
    hm_double4 acc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = hm_double4{0.0, 0.0, 0.0, 0.0};
    double hsq = 0.0, wsq[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int c = 0; c < kMS - 1; ++c)
        if (c < nk) issue(c, c);
    // The K loop, in four copies: with or without h's squares (the waves of
    // expert block 0 write them) and W's squares (wnorm); the choice is made
    // once per wave, outside the loop (every copy takes the same barriers).
    auto kloop = [&](auto hs, auto ws) __attribute__((always_inline)) {
        constexpr bool HS = decltype(hs)::value, WS = decltype(ws)::value;
        for (int c = 0; c < nk; ++c) {
            const int slot = c % kMS;
            if (c + kMS - 2 < nk) wait_vmcnt<(kMS - 2) * 2>();
            else wait_vmcnt<0>();
            lds_barrier();  // chunk c landed for every wave; chunk c-1 fully read
            if (c + kMS - 1 < nk) issue((c + kMS - 1) % kMS, c + kMS - 1);
            const char* st = ring[slot];
            if (tb == 0) {
                // the first token block also writes the chunk of W transposed:
                // lane l -> expert e0 + 16*wave + l/4, k 4*(l%4) .. +3
                const int ex = 16 * wave + (lane >> 2), kq = 4 * (lane & 3);
                const float* sw = reinterpret_cast<const float*>(st) + kq * kME + ex;
                *reinterpret_cast<float4*>(wt + (int64_t)(e0 + ex) * hidden + kb + 16 * c + kq) =
                    make_float4(sw[0], sw[kME], sw[2 * kME], sw[3 * kME]);
            }
            const float4 a = *reinterpret_cast<const float4*>(st + kMW + (16 * wave + i) * 64 + 16 * g);
            float4 wv[4];
    #pragma unroll
            for (int j = 0; j < 4; ++j)
                wv[j] = *reinterpret_cast<const float4*>(st + (4 * g + j) * 256 + 16 * i);
            const double ad[4] = {live ? (double)a.x : 0.0, live ? (double)a.y : 0.0,
                                  live ? (double)a.z : 0.0, live ? (double)a.w : 0.0};
    #pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (HS) hsq = __builtin_fma(ad[j], ad[j], hsq);
                const double bd[4] = {(double)wv[j].x, (double)wv[j].y, (double)wv[j].z,
                                      (double)wv[j].w};
    #pragma unroll
                for (int q = 0; q < 4; ++q)
                    acc[q] = __builtin_amdgcn_mfma_f64_16x16x4f64(ad[j], bd[q], acc[q], 0, 0, 0);
                if constexpr (WS) {
    #pragma unroll
                    for (int q = 0; q < 4; ++q) wsq[q] = __builtin_fma(bd[q], bd[q], wsq[q]);
                }
            }
        }
    };
    if (eb == 0) {
        if (wnorm) kloop(std::true_type{}, std::true_type{});
        else kloop(std::true_type{}, std::false_type{});
    } else {
        if (wnorm) kloop(std::false_type{}, std::true_type{});
        else kloop(std::false_type{}, std::false_type{});
    }
    // partial logits: register r of lane (g, i) holds D[g + 4r][i], i.e.
    // token t0 + g + 4r, experts e0 + 4i .. +3
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int t = t0 + g + 4 * r;
        if (t < tokens) {
            double* o = part + ((int64_t)sp * tokens + t) * experts + e0 + 4 * i;
            *reinterpret_cast<double2*>(o) = double2{acc[0][r], acc[1][r]};
            *reinterpret_cast<double2*>(o + 2) = double2{acc[2][r], acc[3][r]};
        }
    }
    // norms over this range: the four k-slots of a token / expert are the
    // lanes i, i + 16, i + 32, i + 48
    hsq += __shfl_xor(hsq, 16, HM_WAVE);
    hsq += __shfl_xor(hsq, 32, HM_WAVE);
    // (the norms themselves: their square roots, once here rather than for
    // every logit in the select kernel)
    if (eb == 0 && g == 0 && live) hnorm_r[(int64_t)sp * tokens + tok] = sqrt(hsq);
    if (wnorm) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            wsq[q] += __shfl_xor(wsq[q], 16, HM_WAVE);
            wsq[q] += __shfl_xor(wsq[q], 32, HM_WAVE);
        }
        if (g == 0) {
            double* o = wnorm_r + (int64_t)sp * experts + e0 + 4 * i;
            *reinterpret_cast<double2*>(o) = double2{sqrt(wsq[0]), sqrt(wsq[1])};
            *reinterpret_cast<double2*>(o + 2) = double2{sqrt(wsq[2]), sqrt(wsq[3])};
        }
    }
}

// Fallback chains of the split select.  A wave's uncertified logits are
// taken kFN at a time: lane f < kFN runs the reference's chain (k
// ascending) for the f-th of them.  The whole wave stages the next
// kFK-long piece of their W columns (rows of the transposed copy the
// matrix-core kernel wrote) and of the token's h row into LDS with 16-byte
// DMA (double-buffered), then forms that piece's exact products
// double(h_k) * double(w_k) (48-bit, exact in FP64) for both chains in an
// LDS product buffer, so a chain step is one dependent FP64 add,
// acc + p_k == fma(h_k, w_k, acc), with no conversions on its path.
constexpr int kFK = 128;                        // k per staged piece
constexpr int kFN = 2;                          // chains per round
constexpr int kFS = 3;                          // pieces in the staging ring (LDS: four
                                                // workgroups per CU)
constexpr int kFBuf = 4 * kFK * 4;              // one buffer: 2 columns, h, pad (2 KB)
constexpr int kFProd = kFN * kFK * 8;           // products of one piece (2 KB)
constexpr int kFWave = kFS * kFBuf + kFProd;    // fallback LDS per wave
constexpr int kFDma = 2;                        // 16-byte DMA instructions per piece
static_assert(kFK == 2 * HM_WAVE && kFN == 2, "half a wave per staged row piece");
static_assert(kFS == 3, "the staging waits below count three pieces");

__device__ __forceinline__ void fallback_issue(char* buf, const float* __restrict__ hrow,
                                               const float* __restrict__ wt, int64_t hidden,
                                               int64_t k0, const int (&fe)[kFN], int lane) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this buffer's last reads are done
    const int half = lane >> 5;
    const int64_t k = min(k0 + 4 * (lane & 31), hidden - 4);  // past the end: unused
    // lanes 0-31: column 0, lanes 32-63: column 1; then h twice (the second
    // copy lands in the pad)
    dma16(wt + (int64_t)fe[half] * hidden + k, buf);
    dma16(hrow + k, buf + 2 * 4 * kFK);
}

// The idx-th set bit over the masks need[0..EPL) in (j, lane) order:
// its lane and j.
template <int EPL>
__device__ __forceinline__ void locate_fallback(const unsigned long long (&need)[EPL], int idx,
                                                int& owner, int& slot) {
    int jj = 0;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        const int c = __popcll(need[j]);
        if (jj == j && idx >= c) { idx -= c; jj = j + 1; }
    }
    unsigned long long m = need[0];
#pragma unroll
    for (int j = 0; j < EPL; ++j) if (j == jj) m = need[j];
    for (int b = 0; b < idx; ++b) m &= m - 1;
    owner = __ffsll((long long)m) - 1;
    slot = jj;
}

template <int EPL>
__global__ __launch_bounds__(kBlock) void router_select_split_kernel(
    const float* __restrict__ h, const float* __restrict__ wt, const double* __restrict__ part,
    const double* __restrict__ hnorm_r, const double* __restrict__ wnorm_r, int64_t tokens,
    int64_t hidden, int64_t experts, int splits, int32_t top_k, uint32_t flags,
    float* __restrict__ logits, uint32_t* __restrict__ ids, float* __restrict__ scores,
    int32_t* status, hm_row_quant xq, int32_t* __restrict__ hist) {
    // per wave: experts floats for the sequential softmax sum, then the
    // fallback chains' staging ring and products (kFWave, 16-byte aligned)
    extern __shared__ __attribute__((aligned(16))) char dyn_lds[];
    const int lane = threadIdx.x & (HM_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / HM_WAVE);
    const int64_t t = (int64_t)blockIdx.x * (kBlock / HM_WAVE) + wave;
    if (t >= tokens) return;
    const int64_t seq_stride = ((experts * 4 + 15) / 16) * 16;
    float* seq_lds = reinterpret_cast<float*>(dyn_lds);  // indexed by wave * experts
    char* fb = dyn_lds + (kBlock / HM_WAVE) * seq_stride + (int64_t)wave * kFWave;
    double* fprod = reinterpret_cast<double*>(fb + kFS * kFBuf);
    const double u = 0x1p-53;
    const double n = (double)hidden, m = (double)(hidden / splits);
    // the range form's bound (derived above router_mfma_kernel)
    const double g2 = 2.0 * m * u / (1.0 - 2.0 * m * u);
    const double cu = u / (1.0 - u) / (1.0 - n * u / (1.0 - u)) * m;
    // (all loads of the range sums go out before the additions:
    // unconditional loads from clamped ranges, so that no branch splits
    // them from their uses)
    double hr[kMaxSplits];
#pragma unroll
    for (int sp = 0; sp < kMaxSplits; ++sp)
        hr[sp] = hnorm_r[(int64_t)min(sp, splits - 1) * tokens + t];
    float v[EPL];
    bool valid[EPL];
    unsigned long long need[EPL];
    int total = 0;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        const int64_t e = lane + (int64_t)HM_WAVE * j;
        valid[j] = e < experts;
        bool nd = false;
        v[j] = 0.0f;
        if (valid[j]) {
            double pa[kMaxSplits], pw[kMaxSplits];
#pragma unroll
            for (int sp = 0; sp < kMaxSplits; ++sp) {
                const int64_t sc = min(sp, splits - 1);
                pa[sp] = part[(sc * tokens + t) * experts + e];
                pw[sp] = wnorm_r[sc * experts + e];
            }
            // S' (the ranges' partials added in order), the sums of |S'|
            // before (pre) and after (post) each addition, and of the
            // ranges' norm products
            double a = 0.0, pre = 0.0, post = 0.0, nsum = 0.0;
#pragma unroll
            for (int sp = 0; sp < kMaxSplits; ++sp) {
                if (sp < splits) {
                    pre += fabs(a);
                    a += pa[sp];
                    post += fabs(a);
                    nsum += hr[sp] * pw[sp];
                }
            }
            // nsum bounds sum_r sum_{k in r} |p_k| (Cauchy-Schwarz per range;
            // the computed norms err by at most gamma_m relative, covered by
            // the final inflation)
            const double d = g2 * nsum + u * post;
            const double bc = (cu * (pre + (double)splits * d + nsum) + d) * (1.0 + 0x1p-20);
            const double lo = a - bc, hi = a + bc;
            nd = !(isfinite(lo) && isfinite(hi) &&
                   __float_as_uint((float)lo) == __float_as_uint((float)hi));
            v[j] = (float)a;
        }
        need[j] = __ballot(nd);
        total += __popcll(need[j]);
    }
    const float* hrow = h + t * hidden;
    if (total > 0 && hidden % (kNB * 16) == 0) {
        // Second level: the decode path's block form and its much tighter
        // bound, two logits at a time, lane 32*half + j summing block j of
        // the half's logit (b = H/32 terms, sequentially from +0) beside
        // R_j and Q_j; the block sums are then chained in order.  Logits it
        // settles leave the list; the rest take the full chain below.
        const int half = lane >> 5, bj = lane & 31;
        const int64_t bw = hidden / kNB;
        bool left[EPL];
#pragma unroll
        for (int j = 0; j < EPL; ++j) left[j] = (need[j] >> lane) & 1ull;
        for (int done = 0; done < total; done += 2) {  // wave-uniform
            const int idx = min(done + half, total - 1);
            int owner, js;
            locate_fallback<EPL>(need, idx, owner, js);
            const int64_t e = owner + (int64_t)HM_WAVE * js;
            const float* hp = hrow + bj * bw;
            const float* wp = wt + e * hidden + bj * bw;
            double acc = 0.0, rs = 0.0, qs = 0.0;
            // 16 k per step; the next step's loads go out before this step's
            // chains (the last step loads its own chunk again)
            float4 hv[4], wv[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                hv[q] = *reinterpret_cast<const float4*>(hp + 4 * q);
                wv[q] = *reinterpret_cast<const float4*>(wp + 4 * q);
            }
            for (int64_t k0 = 0; k0 < bw; k0 += 16) {
                const int64_t kn = k0 + 16 < bw ? k0 + 16 : k0;
                float4 hn[4], wn[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    hn[q] = *reinterpret_cast<const float4*>(hp + kn + 4 * q);
                    wn[q] = *reinterpret_cast<const float4*>(wp + kn + 4 * q);
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float hq[4] = {hv[q].x, hv[q].y, hv[q].z, hv[q].w};
                    const float wq[4] = {wv[q].x, wv[q].y, wv[q].z, wv[q].w};
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const double hk = (double)hq[r], wk = (double)wq[r];
                        acc = __builtin_fma(hk, wk, acc);  // == acc + hk * wk
                        rs += fabs(acc);
                        qs = __builtin_fma(fabs(hk), fabs(wk), qs);
                    }
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) { hv[q] = hn[q]; wv[q] = wn[q]; }
            }
            const double cj = block_c_term(rs, qs, hidden);
            double a = 0.0, sa = 0.0, sc = 0.0;
#pragma unroll
            for (int j = 0; j < kNB; ++j) {
                a += __shfl(acc, 32 * half + j, HM_WAVE);
                sa += fabs(a);
                sc += __shfl(cj, 32 * half + j, HM_WAVE);
            }
            const bool ok = block_sums_settle(a, sa, sc, hidden);
            // the owners of this pass's logits take the settled values
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                const int o = __shfl(owner, 32 * hf, HM_WAVE);
                const int jo = __shfl(js, 32 * hf, HM_WAVE);
                const bool okh = __shfl((int)ok, 32 * hf, HM_WAVE) != 0;
                const float vh = __shfl((float)a, 32 * hf, HM_WAVE);
                if (okh && lane == o && (hf == 0 || done + 1 < total)) {
#pragma unroll
                    for (int j = 0; j < EPL; ++j) if (j == jo) { v[j] = vh; left[j] = false; }
                }
            }
        }
        total = 0;
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            need[j] = __ballot(left[j]);
            total += __popcll(need[j]);
        }
    }
    for (int done = 0; done < total; done += kFN) {  // wave-uniform
        // the experts of fallbacks done .. done + kFN - 1 (in (j, lane)
        // order; slots past the last repeat it)
        int fe[kFN];
        int owner[kFN], slot[kFN];
#pragma unroll
        for (int f = 0; f < kFN; ++f) {
            locate_fallback<EPL>(need, min(done + f, total - 1), owner[f], slot[f]);
            fe[f] = owner[f] + HM_WAVE * slot[f];
        }
        const int nf = min(kFN, total - done);
        double acc = 0.0;
        const int64_t pieces = (hidden + kFK - 1) / kFK;
#pragma unroll
        for (int c = 0; c < kFS - 1; ++c)
            if (c < pieces) fallback_issue(fb + c * kFBuf, hrow, wt, hidden, c * kFK, fe, lane);
        for (int64_t c = 0; c < pieces; ++c) {
            char* cur = fb + (c % kFS) * kFBuf;
            // the piece kFS - 1 ahead goes into the buffer piece c - 1 used
            // (fallback_issue waits for its reads)
            if (c + kFS - 1 < pieces)
                fallback_issue(fb + ((c + kFS - 1) % kFS) * kFBuf, hrow, wt, hidden,
                               (c + kFS - 1) * kFK, fe, lane);
            // piece c has landed once at most the pieces issued after it are
            // in flight (each piece is kFDma loads; nothing else is loaded here)
            const int64_t after = min((int64_t)kFS - 1, pieces - 1 - c);
            if (after >= 2) wait_vmcnt<2 * kFDma>();
            else if (after == 1) wait_vmcnt<kFDma>();
            else wait_vmcnt<0>();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            const int kc = (int)min((int64_t)kFK, hidden - c * kFK);  // a multiple of 16
            {
                // the piece's products: lane l forms k = 2l, 2l+1 of both chains
                const float2 hv = reinterpret_cast<const float2*>(cur + 2 * 4 * kFK)[lane];
                const float2 w0 = reinterpret_cast<const float2*>(cur)[lane];
                const float2 w1 = reinterpret_cast<const float2*>(cur + 4 * kFK)[lane];
                const double h0 = (double)hv.x, h1 = (double)hv.y;
                reinterpret_cast<double2*>(fprod)[lane] = double2{h0 * (double)w0.x, h1 * (double)w0.y};
                reinterpret_cast<double2*>(fprod + kFK)[lane] = double2{h0 * (double)w1.x, h1 * (double)w1.y};
            }
            // (one wave's LDS accesses complete in order: the chain lanes'
            // reads below see every lane's products)
            if (lane < nf) {
                // 16 products per step, the next step's read out while this
                // one's are added (kc is a multiple of 16)
                const double2* pp = reinterpret_cast<const double2*>(fprod + lane * kFK);
                double2 pa[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) pa[q] = pp[q];
                for (int kk = 0; kk < kc; kk += 16) {
                    const int nx = kk + 16 < kc ? (kk + 16) / 2 : kk / 2;
                    double2 pb[8];
#pragma unroll
                    for (int q = 0; q < 8; ++q) pb[q] = pp[nx + q];
#pragma unroll
                    for (int q = 0; q < 8; ++q) {
                        acc = acc + pa[q].x;
                        acc = acc + pa[q].y;
                    }
#pragma unroll
                    for (int q = 0; q < 8; ++q) pa[q] = pb[q];
                }
            }
            // the products are rewritten for the next piece only after
            // the chains have read them
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
        if (lane < nf && !isfinite(acc)) hm_status_or(status, HM_STATUS_NONFINITE_SCORE);
#pragma unroll
        for (int f = 0; f < kFN; ++f) {
            const double r = __shfl(acc, f, HM_WAVE);
            if (f < nf && lane == owner[f]) {
#pragma unroll
                for (int j = 0; j < EPL; ++j) if (j == slot[f]) v[j] = (float)r;
            }
        }
    }
#pragma unroll
    for (int j = 0; j < EPL; ++j)
        if (valid[j] && logits) logits[t * experts + lane + HM_WAVE * j] = v[j];
    select_token<EPL>(v, valid, lane, wave, t, experts, top_k, flags, ids, scores, status,
                      seq_lds);
    // The permutation's histogram of each 1024-pair chunk (hm_permute's
    // count pass): each lane re-reads the id it has just written.  Integer
    // counts, so the atomics' order does not matter.
    if (hist && lane < top_k) {
        const int64_t pr = t * top_k + lane;
        atomicAdd(&hist[(pr / kPermChunk) * experts + ids[pr]], 1);
    }
    // The token's row in fixed-point digits for the INT8 expert GEMMs (the
    // block's activation quantisation, fused here: this kernel's time is set
    // by a few waves' sequential chains, the rest of the machine is idle).
    if (xq.digits) {
        const int nv = (int)(hidden / 256);
        const hm_dlay lay = hm_dlay_x(xq.limbs, hidden);
        int8_t* d = xq.digits + t * lay.row;
        int32_t* ds = xq.dsum ? xq.dsum + t : nullptr;
        switch (xq.limbs) {
        case 1: hm_quantize_row_wave<1>(hrow, nv, d, lay, xq.scales + t, ds, tokens); break;
        case 2: hm_quantize_row_wave<2>(hrow, nv, d, lay, xq.scales + t, ds, tokens); break;
        default: hm_quantize_row_wave<3>(hrow, nv, d, lay, xq.scales + t, ds, tokens); break;
        }
    }
}

// ---------------------------------------------------------------------------
// A3 permute (src/router/CpuRouterBackend.cpp:140-159).  The reference
// appends (t, score) to group ids[t,r] walking tokens in ascending order and
// then sorts the groups by id: a stable counting sort of the T*k pairs in
// token-major order.  Here the pairs are cut into chunks of 1024:
//   permute_count_kernel    one workgroup per chunk: the chunk's expert
//                           histogram (LDS, order-free) -> hist[chunk][E]
//   permute_scatter_kernel  one workgroup per chunk: offsets[e] (exclusive
//                           scan of the column sums), the chunk's base per
//                           expert (lower chunks' counts), and each pair's
//                           rank among the chunk's earlier pairs of the same
//                           expert (shuffles inside a wave, per-wave counts
//                           across waves) -> its grouped position.
// No global atomics; every position is a pure function of the ids.  A single
// chunk (decode) needs no histogram pass.
// ---------------------------------------------------------------------------
constexpr int kPermThreads = kPermChunk;
constexpr int kPermWaves = kPermThreads / 64;

// Ids past the expert count (a caller's bad input, or the placeholders a
// failed routing leaves for the status word to report) count as the last
// expert, as in permute_small: every LDS index and grouped position stays in
// range whatever the ids hold.
__device__ __forceinline__ int clamp_expert(uint32_t e, int64_t experts) {
    return e < (uint64_t)experts ? (int)e : (int)experts - 1;
}

__global__ __launch_bounds__(kPermThreads) void permute_count_kernel(
    const uint32_t* __restrict__ ids, int64_t pairs, int64_t experts, int32_t* __restrict__ hist) {
    __shared__ int h[1024];
    const int tid = threadIdx.x;
    for (int i = tid; i < experts; i += kPermThreads) h[i] = 0;
    __syncthreads();
    const int64_t p = (int64_t)blockIdx.x * kPermThreads + tid;
    if (p < pairs) atomicAdd(&h[clamp_expert(ids[p], experts)], 1);
    __syncthreads();
    for (int i = tid; i < experts; i += kPermThreads) hist[(int64_t)blockIdx.x * experts + i] = h[i];
}

__global__ __launch_bounds__(kPermThreads) void permute_scatter_kernel(
    const uint32_t* __restrict__ ids, const float* __restrict__ scores, int64_t pairs,
    int32_t top_k, int64_t experts, const int32_t* __restrict__ hist, int64_t chunks,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ perm_tokens, float* __restrict__ perm_weights,
    int32_t* __restrict__ slots) {
    __shared__ int base[1024];                 // this chunk's first position per expert
    __shared__ int wcount[kPermWaves][1024];   // per-wave counts (this chunk)
    __shared__ int scan_w[kPermWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t c = blockIdx.x;
    const int64_t p = c * kPermThreads + tid;
    const int e = p < pairs ? clamp_expert(ids[p], experts) : -1;
    for (int i = tid; i < kPermWaves * experts; i += kPermThreads)
        wcount[i / experts][i % experts] = 0;
    __syncthreads();
    if (e >= 0) atomicAdd(&wcount[wave][e], 1);
    __syncthreads();
    // column sums over chunks (total per expert) and the lower chunks' part
    int total = 0, before = 0;
    if (tid < experts) {
        if (hist) {
            // (eight loads in flight per round)
            for (int64_t c0 = 0; c0 < chunks; c0 += 8) {
                int v[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) v[q] = c0 + q < chunks ? hist[(c0 + q) * experts + tid] : 0;
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    total += v[q];
                    if (c0 + q < c) before += v[q];
                }
            }
        } else {
            for (int w = 0; w < kPermWaves; ++w) total += wcount[w][tid];
        }
    }
    // exclusive scan of the totals over experts (one value per thread)
    int incl = total;
#pragma unroll
    for (int sft = 1; sft < 64; sft <<= 1) {
        const int o = __shfl_up(incl, sft, 64);
        if (lane >= sft) incl += o;
    }
    if (lane == 63) scan_w[wave] = incl;
    __syncthreads();
    int wbase = 0;
    for (int w = 0; w < wave; ++w) wbase += scan_w[w];
    const int offset = wbase + incl - total;
    if (tid < experts) {
        base[tid] = offset + before;
        if (c == 0) {
            counts[tid] = total;
            offsets[tid] = offset;
            if (tid == experts - 1) offsets[experts] = offset + total;
        }
    }
    __syncthreads();
    if (e < 0) return;
    // rank among the chunk's earlier pairs of the same expert: earlier
    // waves' counts, then the wave's earlier lanes with the same id (their
    // mask from one ballot per id bit over the wave's remaining lanes;
    // pairs past the end have left and come after every live pair)
    int rank = 0;
    for (int w = 0; w < wave; ++w) rank += wcount[w][e];
    unsigned long long same = __ballot(true);
    for (int b = 0; (1 << b) < experts; ++b) {
        const bool bit = (e >> b) & 1;
        const unsigned long long m = __ballot(bit);
        same &= bit ? m : ~m;
    }
    rank += __popcll(same & ((1ull << lane) - 1));
    const int pos = base[e] + rank;
    perm_tokens[pos] = (int32_t)(p / top_k);
    perm_weights[pos] = scores[p];
    slots[p] = pos;
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
// distinct, so ranking them gives that order.  One workgroup per token; each
// thread owns 4-element column groups (float4 loads and stores).  Optional
// residual added last (TransformerBlock.cpp:101-104).
// ---------------------------------------------------------------------------
constexpr int kMaxTopK = 64;

__global__ __launch_bounds__(kBlock) void combine_kernel(
    const float* __restrict__ y, const uint32_t* __restrict__ ids,
    const int32_t* __restrict__ slots, const float* __restrict__ scores,
    int64_t tokens, int32_t top_k, int64_t width,
    const float* __restrict__ residual, float* __restrict__ out) {
    __shared__ int64_t srow[kMaxTopK];
    __shared__ float sw[kMaxTopK];
    const int64_t t = blockIdx.x;
    const int tid = threadIdx.x;
    if (tid < top_k) {  // rank of this pair among the token's ids, ascending
        const uint32_t id = ids[t * top_k + tid];
        int rank = 0;
        for (int r = 0; r < top_k; ++r) rank += ids[t * top_k + r] < id;
        srow[rank] = slots[t * top_k + tid];
        sw[rank] = scores[t * top_k + tid];
    }
    __syncthreads();
    if ((width & 3) == 0) {
        const int64_t w4 = width >> 2;
        // two column groups per thread per pass: sixteen rows' float4 loads
        // in flight before the adds (ascending order per column); y is read
        // once, with the streaming hint
        for (int64_t i0 = tid; i0 < w4; i0 += 2 * kBlock) {
          float4 res[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) res[h] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
          for (int r0 = 0; r0 < top_k; r0 += 8) {
            float4 v[2][8];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int64_t i = i0 + h * kBlock;
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    v[h][q] = r0 + q < top_k && i < w4
                                  ? hm_load_stream(
                                        reinterpret_cast<const float4*>(y + srow[r0 + q] * width) + i)
                                  : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                float4 acc = res[h];
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    if (r0 + q < top_k) {
                        const float wv = sw[r0 + q];
                        acc.x = __fadd_rn(acc.x, __fmul_rn(wv, v[h][q].x));
                        acc.y = __fadd_rn(acc.y, __fmul_rn(wv, v[h][q].y));
                        acc.z = __fadd_rn(acc.z, __fmul_rn(wv, v[h][q].z));
                        acc.w = __fadd_rn(acc.w, __fmul_rn(wv, v[h][q].w));
                    }
                }
                res[h] = acc;
            }
          }
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int64_t i = i0 + h * kBlock;
            if (i >= w4) break;
            float4 acc = res[h];
            if (residual) {
                const float4 rv = reinterpret_cast<const float4*>(residual + t * width)[i];
                acc.x = __fadd_rn(rv.x, acc.x);
                acc.y = __fadd_rn(rv.y, acc.y);
                acc.z = __fadd_rn(rv.z, acc.z);
                acc.w = __fadd_rn(rv.w, acc.w);
            }
            reinterpret_cast<float4*>(out + t * width)[i] = acc;
          }
        }
        return;
    }
    for (int64_t i = tid; i < width; i += kBlock) {
        float acc = 0.0f;
        for (int r = 0; r < top_k; ++r) acc = __fadd_rn(acc, __fmul_rn(sw[r], y[srow[r] * width + i]));
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

// hm_rmsnorm's launch; force_seq: every row takes the sequential sum of
// squares (HM_EXEC_ROUTE_SEQUENTIAL through hm_moe_layer_forward).
int hm_launch_rmsnorm(const float* x, const float* gamma, float* y, int64_t rows,
                      int64_t width, float eps, bool force_seq, void* stream) {
    HM_REQUIRE(x && gamma && y && rows >= 0 && width > 0);
    HM_REQUIRE(std::isfinite(eps) && eps > 0.0f);  // RMSNorm.cpp:22
    HM_REQUIRE(width <= 16384);                     // row staged in LDS
    if (rows == 0) return HM_OK;
    HM_REQUIRE(rows <= INT_MAX);
    const bool aligned = ((uintptr_t)x | (uintptr_t)gamma | (uintptr_t)y) % 16 == 0;
    if (aligned && width % 256 == 0 && width / 256 <= 16) {
        const unsigned grid = (unsigned)((rows + kBlock / HM_WAVE - 1) / (kBlock / HM_WAVE));
        const size_t lds = (size_t)(kBlock / HM_WAVE) * 512 * sizeof(double);
        const hipStream_t s = hm_stream(stream);
        const int fs = force_seq ? 1 : 0;
        switch (width / 256) {
#define HM_RMS_CASE(v) \
    case v: hipLaunchKernelGGL(rmsnorm_wave_kernel<v>, dim3(grid), dim3(kBlock), lds, s, x, gamma, y, rows, eps, fs); break;
            HM_RMS_CASE(1) HM_RMS_CASE(2) HM_RMS_CASE(3) HM_RMS_CASE(4) HM_RMS_CASE(5) HM_RMS_CASE(6)
            HM_RMS_CASE(7) HM_RMS_CASE(8) HM_RMS_CASE(9) HM_RMS_CASE(10) HM_RMS_CASE(11)
            HM_RMS_CASE(12) HM_RMS_CASE(13) HM_RMS_CASE(14) HM_RMS_CASE(15) HM_RMS_CASE(16)
#undef HM_RMS_CASE
        }
        HM_LAUNCHED();
        return HM_OK;
    }
    hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(kBlock),
                       (size_t)width * sizeof(float), hm_stream(stream), x, gamma,
                       y, width, eps, force_seq ? 1 : 0);
    HM_LAUNCHED();
    return HM_OK;
}

extern "C" {

int hm_rmsnorm(const float* x, const float* gamma, float* y, int64_t rows,
               int64_t width, float eps, void* stream) {
    return hm_launch_rmsnorm(x, gamma, y, rows, width, eps, false, stream);
}


// Route workspace: the logits [T x E] floats (rounded up to 256 bytes),
// then for decode batches (T <= kDecodeTokens) the block partials
// [T x E x 2 x kNB] doubles, and for prefill batches with E % 64 == 0 the
// matrix-core range partials [S x T x E] doubles, W transposed [E x H]
// floats, row norms [S x T] and column norms [S x E] doubles
// (S = prefill_splits).
constexpr int64_t kDecodeTokens = 16;

static size_t route_logits_bytes(int64_t tokens, int64_t experts) {
    return ((size_t)tokens * (size_t)experts * sizeof(float) + 255) & ~(size_t)255;
}

// K ranges of the prefill logits: enough workgroups (>= 512) to give every
// SIMD two waves; H must also be a multiple of 16 per range (the launcher
// halves S until it is).
static int prefill_splits(int64_t tokens, int64_t experts) {
    const int64_t base = ((tokens + kMT - 1) / kMT) * (experts / kME);
    int sp = 1;
    while (sp < kMaxSplits && base * sp < 512) sp *= 2;
    return sp;
}

size_t hm_route_workspace_bytes(int64_t tokens, int64_t hidden, int64_t experts) {
    if (tokens < 0 || experts <= 0 || hidden <= 0) return 0;
    if (tokens > kDecodeTokens) {
        size_t b = route_logits_bytes(tokens, experts);
        if (experts % kME == 0) {
            const size_t sp = (size_t)prefill_splits(tokens, experts);
            b += sp * ((size_t)tokens * (size_t)experts + (size_t)tokens + (size_t)experts) *
                     sizeof(double) +
                 (size_t)experts * (size_t)hidden * sizeof(float);
        }
        return b;
    }
    return route_logits_bytes(tokens, experts) +
           (size_t)tokens * (size_t)experts * kNB * 2 * sizeof(double);
}

}  // extern "C"

// The decode router's two launches.  With `fused`, the select kernel also
// forms the expert groups (the workgroup that finishes last) and the
// partial kernel zeroes the fused step's completion counters first.
static int launch_decode_router(const float* h, const float* w, int64_t tokens, int64_t hidden,
                                int64_t experts, int32_t top_k, uint32_t flags, float* logits,
                                uint32_t* ids, float* scores, int32_t* status, void* route_ws,
                                const hm_decode_fusion* fused, const hm_norm_fold* norm,
                                const hm_row_quant* xq, void* stream, bool select = true) {
    const hm_row_quant q = xq && fused ? *xq : hm_row_quant{nullptr, nullptr, nullptr, 0};
    const int epl = (int)((experts + HM_WAVE - 1) / HM_WAVE);
    // fused: one token per workgroup, its logit rows shared out over up to
    // four waves; else four tokens (waves) per workgroup
    const int nw = !fused ? 4 : epl <= 1 ? 1 : epl <= 2 ? 2 : 4;
    const dim3 sgrid((unsigned)(fused ? tokens : (tokens + 3) / 4));
    const size_t seq_bytes = (size_t)nw * experts * sizeof(float);
    double* part = reinterpret_cast<double*>(static_cast<char*>(route_ws) +
                                             route_logits_bytes(tokens, experts));
    const dim3 pgrid((unsigned)kNB, (unsigned)((experts + HM_WAVE - 1) / HM_WAVE),
                     (unsigned)tokens);
    const hm_norm_fold nf = norm ? *norm : hm_norm_fold{nullptr, nullptr, 0.0f, 0};
    hipLaunchKernelGGL(router_partial_kernel, pgrid, dim3(HM_WAVE),
                       norm ? (size_t)hidden * sizeof(float) : 0, hm_stream(stream), h, w,
                       (int)hidden, (int)experts, part, fused ? fused->counters : nullptr,
                       fused ? fused->n_counters : 0, nf);
    HM_LAUNCHED();
    if (!select) return HM_OK;
    // the select kernel's fallback chains read the normalised rows
    if (norm) h = norm->x_out;
#define HM_SELECTP(N, F, W)                                                                \
    hipLaunchKernelGGL((router_select_partial_kernel<N, F, W, F>), sgrid, dim3(W * HM_WAVE), \
                       seq_bytes, hm_stream(stream), h, w, part, tokens, hidden, experts,    \
                       top_k, flags, logits, ids, scores, status,                            \
                       F ? fused->counters : nullptr, F ? fused->counts : nullptr,           \
                       F ? fused->offsets : nullptr, F ? fused->perm_tokens : nullptr,       \
                       F ? fused->perm_weights : nullptr, F ? fused->slots : nullptr, q)
#define HM_SELECTP2(N)                                  \
    do {                                                \
        if (!fused) HM_SELECTP(N, false, 4);            \
        else if (nw == 1) HM_SELECTP(N, true, 1);       \
        else if (nw == 2) HM_SELECTP(N, true, 2);       \
        else HM_SELECTP(N, true, 4);                    \
    } while (0)
    if (epl <= 1) HM_SELECTP2(1);
    else if (epl <= 2) HM_SELECTP2(2);
    else if (epl <= 4) HM_SELECTP2(4);
    else if (epl <= 8) HM_SELECTP2(8);
    else HM_SELECTP2(16);
#undef HM_SELECTP2
#undef HM_SELECTP
    HM_LAUNCHED();
    return HM_OK;
}

// One-token decode with the select inside the gate/up launch
// (select_gateup_kernel): the shapes it takes -- an INT8 layer whose
// gate/up the slice kernel covers (the token row in LDS, K tiles within four
// loads per wave), at most 8 rows of 64 logits, the partial kernel's H.
bool hm_select_gateup_ok(const hm_layer* L, int32_t top_k) {
    const int64_t KT = hm_pad32(L->hidden) / 32;
    // (E <= 128: the kernel's LDS holds two rows of block partials; H <= 2 x
    // 4 x 512 floats: the token row in two float4 per thread)
    return L->dtype == HM_DTYPE_INT8 && L->experts <= 2 * HM_WAVE && top_k >= 1 &&
           top_k <= L->experts && top_k <= kMaxTopK && L->hidden % kNB == 0 &&
           L->hidden <= 8 * kGvThreads && KT <= 16 * kGsQ && L->intermediate % 8 == 0;
}

// The first launch of such a step: the router partials (router_partial_kernel,
// which also zeroes the step's counters and, with `norm`, folds the RMSNorm
// in and writes norm->x_out).
int hm_route_partials_decode(const float* h, const float* w, int64_t hidden, int64_t experts,
                             int32_t top_k, uint32_t flags, int32_t* status, void* route_ws,
                             const hm_decode_fusion* fused, const hm_norm_fold* norm,
                             void* stream) {
    HM_REQUIRE(h && w && route_ws && fused && fused->counters && experts > 0 && hidden > 0);
    HM_REQUIRE(!norm || (norm->gamma && norm->x_out && std::isfinite(norm->eps) &&
                         norm->eps > 0.0f && hidden <= 16384));
    if (experts > 1024 || hidden % kNB != 0 || hidden > INT_MAX) return HM_ERR_UNSUPPORTED;
    return launch_decode_router(h, w, 1, hidden, experts, top_k, flags,
                                static_cast<float*>(route_ws), nullptr, nullptr, status, route_ws,
                                fused, norm, nullptr, stream, false);
}

// The second: select_gateup_kernel.  x: the token row the router read (the
// normalised one when the norm is folded); z [k x I]: SiLU(G) * U of the k
// selected experts' rows in ascending id; ids ... slots: the routing results
// and the groups (hm_route_permute_decode's).  The first kernel of the
// gate/up stage and its last (an armed stage timer brackets it).
int hm_launch_select_gateup(const float* x, const float* w, int32_t top_k, uint32_t flags,
                            uint32_t* ids, float* scores, int32_t* status, void* route_ws,
                            int32_t* counts, int32_t* offsets, int32_t* perm_tokens,
                            float* perm_weights, int32_t* slots, const hm_layer* L, float* z,
                            hipStream_t stream) {
    HM_REQUIRE(x && w && ids && scores && route_ws && counts && offsets && perm_tokens &&
               perm_weights && slots && z);
    if (!hm_select_gateup_ok(L, top_k)) return HM_ERR_UNSUPPORTED;
    const int64_t H = L->hidden, E = L->experts, I = L->intermediate;
    const int64_t KT = hm_pad32(H) / 32;
    float* logits = static_cast<float*>(route_ws);
    const double* part = reinterpret_cast<const double*>(static_cast<char*>(route_ws) +
                                                         route_logits_bytes(1, E));
    const dim3 grid((unsigned)(I / 8), (unsigned)top_k);
    const size_t lds = (size_t)H * sizeof(float);
    const int epl = (int)((E + HM_WAVE - 1) / HM_WAVE);
    const int lj = (int)((KT + kGsQ - 1) / kGsQ + 3) / 4;
#define HM_SG(EPL, LJ)                                                                          \
    HM_STAGE_LAUNCH(true, true, (select_gateup_kernel<EPL, LJ>), grid, dim3(kGvThreads), lds,   \
                    stream, x, w, part, H, E, top_k, flags, logits, ids, scores, status, counts, \
                    offsets, perm_tokens, perm_weights, slots, I,                                \
                    static_cast<const int8_t*>(L->packed), L->scale, L->zero_point, z)
#define HM_SG2(EPL)                                                                             \
    do {                                                                                        \
        if (lj <= 1) HM_SG(EPL, 1);                                                             \
        else if (lj <= 2) HM_SG(EPL, 2);                                                        \
        else HM_SG(EPL, 4);                                                                     \
    } while (0)
    if (epl <= 1) HM_SG2(1);
    else HM_SG2(2);
#undef HM_SG2
#undef HM_SG
    HM_LAUNCHED();
    return HM_OK;
}

// Routing and grouping of a decode batch (T <= 16) in two launches instead
// of hm_router_topk + hm_permute's three; same results.  Counter 0 of
// fused->counters is the select's completion counter; all n_counters are
// zeroed by the first launch.  With `norm`, h is the layer input and the
// router (and norm->x_out) get RMSNorm(h) (hm_rmsnorm's results).
int hm_route_permute_decode(const float* h, const float* w, int64_t tokens, int64_t hidden,
                            int64_t experts, int32_t top_k, uint32_t flags, uint32_t* ids,
                            float* scores, int32_t* status, void* route_ws,
                            const hm_decode_fusion* fused, const hm_norm_fold* norm,
                            const hm_row_quant* xq, bool* quantized, void* stream) {
    if (quantized) *quantized = false;
    HM_REQUIRE(experts > 0 && top_k > 0 && top_k <= experts && fused && fused->counters);
    HM_REQUIRE(h && w && ids && scores && route_ws && tokens > 0 && hidden > 0);
    // (the norm's row copy is hidden floats of LDS, as in hm_rmsnorm)
    HM_REQUIRE(!norm || (norm->gamma && norm->x_out && std::isfinite(norm->eps) &&
                         norm->eps > 0.0f && hidden <= 16384));
    if (experts > 1024 || top_k > kMaxTopK || tokens > kDecodeTokens || hidden % kNB != 0 ||
        tokens * top_k > kSmallPairs || hidden > INT_MAX)
        return HM_ERR_UNSUPPORTED;
    // the select kernel also cuts the rows' activation digits when asked
    // (widths the one-wave row quantisation takes; the rows it reads are the
    // normalised ones when the norm is folded in)
    const hm_row_quant* q =
        xq && xq->digits && xq->scales && xq->limbs >= 1 && xq->limbs <= 3 &&
                hidden % 256 == 0 && hidden / 256 <= kHmQuantMaxV &&
                (uintptr_t)xq->digits % 4 == 0 && (uintptr_t)(norm ? norm->x_out : h) % 16 == 0
            ? xq
            : nullptr;
    const int rc = launch_decode_router(h, w, tokens, hidden, experts, top_k, flags,
                                        static_cast<float*>(route_ws), ids, scores, status,
                                        route_ws, fused, norm, q, stream);
    if (rc == HM_OK && q && quantized) *quantized = true;
    return rc;
}

extern "C" {

__attribute__((visibility("hidden"))) int hm_router_topk_quant(const float* h, const float* w, int64_t tokens,
                         int64_t hidden, int64_t experts, int32_t top_k,
                         uint32_t flags, uint32_t* ids, float* scores,
                         float* logits_out, int32_t* status, void* route_ws,
                         const hm_row_quant* xq, bool* quantized, int32_t* hist,
                         bool* counted, void* stream);

__attribute__((visibility("hidden"))) int hm_permute_counted(const uint32_t* ids, const float* scores, int64_t tokens,
                       int32_t top_k, int64_t experts, int32_t* counts, int32_t* offsets,
                       int32_t* perm_tokens, float* perm_weights, int32_t* slots,
                       void* workspace, bool counted, void* stream);

int hm_router_topk(const float* h, const float* w, int64_t tokens,
                   int64_t hidden, int64_t experts, int32_t top_k,
                   uint32_t flags, uint32_t* ids, float* scores,
                   float* logits_out, int32_t* status, void* route_ws,
                   void* stream) {
    return hm_router_topk_quant(h, w, tokens, hidden, experts, top_k, flags, ids, scores,
                                logits_out, status, route_ws, nullptr, nullptr, nullptr,
                                nullptr, stream);
}

// hm_router_topk, and where the prefill select kernel runs, the rows of h
// quantised into xq's digit planes as well (*quantized tells the caller).
__attribute__((visibility("hidden"))) int hm_router_topk_quant(const float* h, const float* w, int64_t tokens,
                         int64_t hidden, int64_t experts, int32_t top_k,
                         uint32_t flags, uint32_t* ids, float* scores,
                         float* logits_out, int32_t* status, void* route_ws,
                         const hm_row_quant* xq, bool* quantized, int32_t* hist,
                         bool* counted, void* stream) {
    if (quantized) *quantized = false;
    if (counted) *counted = false;
    // RouterConfig::validate (src/router/RouterConfig.cpp:9-22)
    HM_REQUIRE(experts > 0 && top_k > 0 && top_k <= experts);
    HM_REQUIRE(h && w && ids && scores && tokens > 0 && hidden > 0);
    HM_REQUIRE(logits_out || route_ws);
    if (experts > 1024 || top_k > kMaxTopK) return HM_ERR_UNSUPPORTED;
    if (tokens > ((int64_t)1 << 31) / kLT) return HM_ERR_OVERFLOW;
    float* logits = logits_out ? logits_out : static_cast<float*>(route_ws);
    const int epl = (int)((experts + HM_WAVE - 1) / HM_WAVE);
    const dim3 sgrid((unsigned)((tokens + 3) / 4));
    const size_t seq_bytes = (size_t)(kBlock / HM_WAVE) * experts * sizeof(float);
    if (route_ws && tokens <= kDecodeTokens && hidden % kNB == 0 && hidden <= INT_MAX) {
        // decode: certified block partials, then select over the logits
        // formed from them
        return launch_decode_router(h, w, tokens, hidden, experts, top_k, flags, logits, ids,
                                    scores, status, route_ws, nullptr, nullptr, nullptr, stream);
    }
    const bool aligned = ((uintptr_t)h % 16 == 0) && ((uintptr_t)w % 16 == 0);
    if (route_ws && !(flags & HM_EXEC_ROUTE_SEQUENTIAL) && aligned && experts % kME == 0 &&
        hidden % 16 == 0 && hidden <= INT_MAX && tokens <= INT_MAX &&
        (uintptr_t)route_ws % 16 == 0) {
        // prefill: matrix-core range partials, then certify + select
        int sp = prefill_splits(tokens, experts);
        while (sp > 1 && hidden % (16 * sp) != 0) sp /= 2;
        double* part = reinterpret_cast<double*>(static_cast<char*>(route_ws) +
                                                 route_logits_bytes(tokens, experts));
        float* wt = reinterpret_cast<float*>(part + (int64_t)sp * tokens * experts);
        double* hnorm_r = reinterpret_cast<double*>(wt + experts * hidden);
        double* wnorm_r = hnorm_r + (int64_t)sp * tokens;
        const int64_t grid = ((tokens + kMT - 1) / kMT) * (experts / kME) * sp;
        // the chunk histograms of hm_permute, when the caller passes them
        const int64_t chunks = (tokens * top_k + kPermChunk - 1) / kPermChunk;
        int32_t* hc = hist && chunks > 1 && chunks * experts <= INT_MAX ? hist : nullptr;
        if (hc && counted) *counted = true;
        hipLaunchKernelGGL(router_mfma_kernel, dim3((unsigned)grid), dim3(256), 0,
                           hm_stream(stream), h, w, (int)tokens, (int)hidden, (int)experts,
                           (int)(hidden / sp), part, wt, hnorm_r, wnorm_r, hc,
                           hc ? (int)(chunks * experts) : 0);
        HM_LAUNCHED();
        const size_t split_bytes =
            (kBlock / HM_WAVE) * ((((size_t)experts * 4 + 15) / 16) * 16 + (size_t)kFWave);
        hm_row_quant q = {nullptr, nullptr, nullptr, 0};
        if (xq && xq->digits && xq->scales && xq->limbs >= 1 && xq->limbs <= 3 &&
            hidden % 256 == 0 && hidden / 256 <= kHmQuantMaxV &&
            (uintptr_t)xq->digits % 4 == 0) {
            q = *xq;
            if (quantized) *quantized = true;
        }
#define HM_SELECTS(N)                                                                     \
        hipLaunchKernelGGL(router_select_split_kernel<N>, sgrid, dim3(kBlock), split_bytes, \
                           hm_stream(stream), h, wt, part, hnorm_r, wnorm_r, tokens, hidden, experts, \
                           sp, top_k, flags, logits, ids, scores, status, q, hc)
        if (epl <= 1) HM_SELECTS(1);
        else if (epl <= 2) HM_SELECTS(2);
        else if (epl <= 4) HM_SELECTS(4);
        else if (epl <= 8) HM_SELECTS(8);
        else HM_SELECTS(16);
#undef HM_SELECTS
        HM_LAUNCHED();
        return HM_OK;
    }
    if (aligned && experts % kTE == 0 && hidden % kTK == 0) {
        const dim3 grid((unsigned)((tokens + kTT - 1) / kTT), (unsigned)(experts / kTE));
        hipLaunchKernelGGL(router_logits_tile_kernel, grid, dim3(256), 0, hm_stream(stream), h,
                           w, tokens, hidden, experts, logits, status);
    } else {
        const dim3 lgrid((unsigned)((tokens + kLT - 1) / kLT),
                         (unsigned)((experts + kLE - 1) / kLE));
        hipLaunchKernelGGL(router_logits_kernel, lgrid, dim3(kBlock), 0, hm_stream(stream),
                           h, w, tokens, hidden, experts, logits, status);
    }
    HM_LAUNCHED();
#define HM_SELECT(N)                                                                   \
    hipLaunchKernelGGL(router_select_kernel<N>, sgrid, dim3(kBlock), seq_bytes,        \
                       hm_stream(stream), logits, tokens, experts, top_k, flags, ids,  \
                       scores, status)
    if (epl <= 1) HM_SELECT(1);
    else if (epl <= 2) HM_SELECT(2);
    else if (epl <= 4) HM_SELECT(4);
    else if (epl <= 8) HM_SELECT(8);
    else HM_SELECT(16);
#undef HM_SELECT
    HM_LAUNCHED();
    return HM_OK;
}

// Permute workspace: the per-chunk histograms [chunks x E] (none for one
// chunk).
size_t hm_permute_workspace_bytes(int64_t tokens, int32_t top_k, int64_t experts) {
    if (tokens <= 0 || top_k <= 0 || experts <= 0) return 0;
    const int64_t chunks = (tokens * top_k + kPermThreads - 1) / kPermThreads;
    return chunks > 1 ? (size_t)chunks * (size_t)experts * sizeof(int32_t) : 0;
}

int hm_permute(const uint32_t* ids, const float* scores, int64_t tokens,
               int32_t top_k, int64_t experts, int32_t* counts, int32_t* offsets,
               int32_t* perm_tokens, float* perm_weights, int32_t* slots,
               void* workspace, void* stream) {
    return hm_permute_counted(ids, scores, tokens, top_k, experts, counts, offsets,
                              perm_tokens, perm_weights, slots, workspace, false, stream);
}

// hm_permute; `counted`: the workspace already holds the chunk histograms
// (the prefill router's select kernel counted them), so only the scatter runs.
__attribute__((visibility("hidden"))) int hm_permute_counted(const uint32_t* ids, const float* scores, int64_t tokens,
                       int32_t top_k, int64_t experts, int32_t* counts, int32_t* offsets,
                       int32_t* perm_tokens, float* perm_weights, int32_t* slots,
                       void* workspace, bool counted, void* stream) {
    HM_REQUIRE(ids && scores && counts && offsets && perm_tokens && perm_weights && slots);
    HM_REQUIRE(tokens > 0 && top_k > 0 && experts > 0 && top_k <= experts);
    if (experts > 1024) return HM_ERR_UNSUPPORTED;
    if (tokens * top_k > INT_MAX) return HM_ERR_OVERFLOW;
    const int64_t pairs = tokens * top_k;
    const int64_t chunks = (pairs + kPermThreads - 1) / kPermThreads;
    int32_t* hist = nullptr;
    if (chunks > 1) {
        HM_REQUIRE(workspace);
        hist = static_cast<int32_t*>(workspace);
    }
    if (chunks > 1 && !counted) {
        hipLaunchKernelGGL(permute_count_kernel, dim3((unsigned)chunks), dim3(kPermThreads), 0,
                           hm_stream(stream), ids, pairs, experts, hist);
        HM_LAUNCHED();
    }
    hipLaunchKernelGGL(permute_scatter_kernel, dim3((unsigned)chunks), dim3(kPermThreads), 0,
                       hm_stream(stream), ids, scores, pairs, top_k, experts, hist, chunks,
                       counts, offsets, perm_tokens, perm_weights, slots);
    HM_LAUNCHED();
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
    HM_REQUIRE(tokens <= INT_MAX);
    hipLaunchKernelGGL(combine_kernel, dim3((unsigned)tokens), dim3(kBlock), 0,
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
