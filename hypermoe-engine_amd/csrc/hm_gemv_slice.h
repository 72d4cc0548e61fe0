// hm_gemv_slice.h -- the decode gate/up GEMV on 8-column slices (shared by
// hm_gemv.hip's slice kernel and hm_router.hip's one-token select + gate/up
// kernel), with the helpers it needs: the W8A32 GEMV constants, the active
// expert lookup from the routed counts, and the tile-to-float conversion.
#ifndef HM_GEMV_SLICE_H
#define HM_GEMV_SLICE_H

#include "hm_device.h"

namespace {

constexpr int kGvWaves = 8;                 // waves per workgroup
constexpr int kGvThreads = 64 * kGvWaves;
constexpr int kGvRows = 4;                  // activation rows per pass (weights stay in registers)
constexpr int kGvMaxTiles = 16;             // K tiles per wave: K <= 32 * 16 * (waves per projection)
constexpr int kGvAllFloats = 16384;         // s_x of every token's row: T * K32 <= this

typedef int v4i __attribute__((ext_vector_type(4)));

// The slot-th expert (ascending id) with a non-zero group (e = -1 if
// none), its group's first grouped row (the exclusive prefix sum of counts,
// i.e. offsets[e]) and its row count, from the counts hm_load_counts read
// (E <= 64 NG).  Every group is reduced before the search, so no load is
// left in flight past this point (a later wait for its register would also
// wait for every load issued after it).  Every wave computes it
// redundantly.
struct hm_active { int e, g0, rows; };

__device__ __forceinline__ int hm_wave_sum(int v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
    return v;
}

// The counts of the NG 64-expert groups (lane l of group b: expert 64 b + l;
// zero past E), loads only: issue them before other loads, so that their
// wait (in hm_active_expert) does not also wait for those.
template <int NG>
__device__ __forceinline__ void hm_load_counts(const int32_t* __restrict__ counts,
                                               int64_t experts, int (&cnt)[NG]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int b = 0; b < NG; ++b) {
        const int64_t e = (int64_t)b * 64 + lane;
        cnt[b] = counts[e < experts ? e : experts - 1];  // (clamped: no branch per load)
    }
}

template <int NG>
__device__ __forceinline__ hm_active hm_active_expert(int (&cnt)[NG], int64_t experts, int slot) {
    const int lane = threadIdx.x & 63;
    unsigned long long m[NG];
    int tot[NG];
#pragma unroll
    for (int b = 0; b < NG; ++b) {
        if ((int64_t)b * 64 + lane >= experts) cnt[b] = 0;
        m[b] = __ballot(cnt[b] > 0);
        tot[b] = hm_wave_sum(cnt[b]);
    }
    hm_active r{-1, 0, 0};
    int seen = 0, before = 0;
#pragma unroll
    for (int b = 0; b < NG; ++b) {
        const int c = __popcll(m[b]);
        if (r.e < 0 && slot < seen + c) {
            // position of the (slot - seen)-th set bit
            unsigned long long mm = m[b];
            for (int i = 0; i < slot - seen; ++i) mm &= mm - 1;
            const int pos = __ffsll((long long)mm) - 1;
            r.e = b * 64 + pos;
            // (uniform values: read from lane 0, so that they live in SGPRs)
            r.rows = __builtin_amdgcn_readfirstlane(__shfl(cnt[b], pos, 64));
            r.g0 = __builtin_amdgcn_readfirstlane(before + hm_wave_sum(lane < pos ? cnt[b] : 0));
        }
        seen += c;
        before += __builtin_amdgcn_readfirstlane(tot[b]);
    }
    return r;
}

// v where keep, else +0 (bitwise: a select between v and a zero vector
// would be turned into a select between their addresses, which puts v in
// scratch memory)
__device__ __forceinline__ float4 hm_keep_if(float4 v, bool keep) {
    const int m = keep ? -1 : 0;
    return make_float4(__int_as_float(__float_as_int(v.x) & m), __int_as_float(__float_as_int(v.y) & m),
                       __int_as_float(__float_as_int(v.z) & m), __int_as_float(__float_as_int(v.w) & m));
}

// 16 unsigned bytes (after XOR 0x80: u = q + 128) -> 16 floats
__device__ __forceinline__ void tile_to_float(v4i w, float (&f)[16]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t u = (uint32_t)w[q] ^ 0x80808080u;  // v_cvt_f32_ubyte0..3 below
        asm volatile("" : "+v"(u));  // converted where used, not hoisted
        f[4 * q + 0] = (float)(u & 0xffu);
        f[4 * q + 1] = (float)((u >> 8) & 0xffu);
        f[4 * q + 2] = (float)((u >> 16) & 0xffu);
        f[4 * q + 3] = (float)(u >> 24);
    }
}

// ---------------------------------------------------------------------------
// Gate/up of a few tokens (T * K32 <= kGvAllFloats) on 8-column slices:
//   z[g, n] = silu(x_g . Wg[n]) * (x_g . Wu[n]),  x_g = hidden[perm_tokens[g]]
// Workgroup: one active expert (the blockIdx.y-th) x 8 columns (slice
// blockIdx.x: N/8 x slots workgroups, three or more per CU at decode, so
// the weight stream and its dequantising arithmetic spread over every CU).
// As in the fused down kernel, one wave-wide 16-byte load covers four K
// tiles of the slice (lane l: tile l / 16, K half (l / 8) % 2, column
// l % 8); wave (p, q) takes projection p and K quarter q, holds its LJ
// loads in registers and runs the expert's rows past them.  Every token's
// row is in LDS (loaded first, with the counts), grouped row g reads row
// perm_tokens[g].  Sums: per lane in K order, the eight lanes of a column
// in a fixed tree, the quarters in order; then the factored dequantisation
// and SiLU(G)*U as in gemv_kernel.
// ---------------------------------------------------------------------------
constexpr int kGsQ = 4;  // K quarters (waves per projection)

// The slice kernel's work for slice bx of active expert slot by.  PRE: the
// expert is known already (pre: its id, first grouped row, row count and,
// tok >= 0, the one token every row reads; counts and perm_tokens are not
// read) and the caller has staged the token rows in s_x (the dynamic LDS)
// and synchronised the workgroup: the one-token select + gate/up kernel,
// whose workgroups select the experts themselves.  R: rows per pass (the
// weights stay in registers across the passes; one token: R = 1).
struct hm_slice_pre {
    int e, g0, rows, tok;
};

template <int NG, int LJ, bool PRE, int R = kGvRows>
__device__ __forceinline__ void gateup_slice_body(
    unsigned bx, unsigned by, hm_slice_pre pre, const float* __restrict__ x_src,
    const int32_t* __restrict__ perm_tokens, int64_t K, int64_t N, int64_t experts,
    const int8_t* __restrict__ packed, const float* __restrict__ scale,
    const int32_t* __restrict__ zp, const int32_t* __restrict__ counts, int n_tokens,
    float* __restrict__ out) {
    extern __shared__ __attribute__((aligned(16))) float s_x[];      // [T][K32]
    static_assert(R >= 1 && R <= kGvRows, "rows per pass");
    __shared__ float s_red[2][kGsQ][R][8];
    __shared__ float s_xs[kGsQ][R];
    __shared__ unsigned long long s_exp2[32];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int p = wave / kGsQ, q = wave % kGsQ;
    const unsigned long long tab = tid < 32 ? kHmExp2Table[tid] : 0ull;
    // counts, then the token rows (only the slices that exist: a uniform
    // bound per load, no data merged at a join)
    int cnt[NG];
    if constexpr (!PRE) hm_load_counts<NG>(counts, experts, cnt);
    const int64_t K32 = hm_pad32(K), KT = K32 / 32;
    const uint32_t k4 = (uint32_t)(K32 / 4), nx = (uint32_t)n_tokens * k4;
    constexpr int kX = PRE ? 1 : kGvAllFloats / 4 / kGvThreads;
    float4 xa[kX];
#pragma unroll
    for (int u = 0; u < kX; ++u) {
        if (!PRE && (uint32_t)u * kGvThreads < nx) {
            const uint32_t i = min((uint32_t)tid + (uint32_t)u * kGvThreads, nx - 1);
            const uint32_t t = i / k4, k = min(4 * (i % k4), (uint32_t)K - 4);
            xa[u] = *reinterpret_cast<const float4*>(x_src + (int64_t)t * K + k);
        }
    }
    hm_active act;
    if constexpr (PRE) act = hm_active{pre.e, pre.g0, pre.rows};
    else act = hm_active_expert<NG>(cnt, experts, (int)by);
    const int e = act.e;
    if (e < 0) return;  // uniform: every wave computes the same e
    // the token of grouped row g
    auto row_token = [&](int64_t g) __attribute__((always_inline)) -> int64_t {
        if constexpr (PRE) { if (pre.tok >= 0) return pre.tok; }
        return perm_tokens[g];
    };
    const int64_t n0 = 8 * (int64_t)bx;
    const int64_t cb = n0 >> 5;
    const int sl = (int)(n0 & 31) >> 3;
    const int kb0 = (int)(q * KT / kGsQ), nkb = (int)((q + 1) * KT / kGsQ) - kb0;
    const int tq = lane >> 4, kh = (lane >> 3) & 1, col = lane & 7;
    // the x rows to LDS (zero past K) before the weights go out
#pragma unroll
    for (int u = 0; u < kX; ++u) {
        const uint32_t i = (uint32_t)tid + (uint32_t)u * kGvThreads;
        if (!PRE && (uint32_t)u * kGvThreads < nx && i < nx)
            *reinterpret_cast<float4*>(&s_x[4 * i]) = hm_keep_if(xa[u], 4 * (i % k4) < K);
    }
    if (tid < 32) s_exp2[tid] = tab;
    __builtin_amdgcn_sched_barrier(0);
    // the weights: LJ loads of four K tiles (tiles past the quarter re-read
    // its last one and are skipped below)
    const int8_t* wsrc = packed + hm_proj_offset(e, p, K, N) + cb * KT * 1024 + 512 * kh +
                         128 * sl + 16 * col;
    v4i w[LJ];
#pragma unroll
    for (int j = 0; j < LJ; ++j)
        w[j] = *reinterpret_cast<const v4i*>(wsrc + (int64_t)(kb0 + min(4 * j + tq, max(nkb - 1, 0))) * 1024);
    __syncthreads();
    const int64_t g0 = act.g0;
    const int rows = act.rows;
    for (int r0 = 0; r0 < rows; r0 += R) {
        const int nr = min(R, rows - r0);
        int64_t xoff[R];
#pragma unroll
        for (int r = 0; r < R; ++r)
            xoff[r] = (r < nr ? row_token(g0 + r0 + r) : 0) * K32 + 32 * (kb0 + tq) + 16 * kh;
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
        for (int j = 0; j < LJ; ++j) {
            if (4 * j + tq < nkb) {
                float f[16];
                tile_to_float(w[j], f);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    if (r < nr) {
                        const float4* xv = reinterpret_cast<const float4*>(&s_x[xoff[r] + 128 * j]);
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float4 v = xv[i];
                            acc[r] = __builtin_fmaf(v.x, f[4 * i], acc[r]);
                            acc[r] = __builtin_fmaf(v.y, f[4 * i + 1], acc[r]);
                            acc[r] = __builtin_fmaf(v.z, f[4 * i + 2], acc[r]);
                            acc[r] = __builtin_fmaf(v.w, f[4 * i + 3], acc[r]);
                        }
                    }
                }
            }
        }
        // the eight lanes of each column: K halves, then the four tiles
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float a = acc[r];
            a += __shfl_xor(a, 8, 64);
            a += __shfl_xor(a, 16, 64);
            a += __shfl_xor(a, 32, 64);
            if (lane < 8) s_red[p][q][r][lane] = a;
        }
        // the rows' sums over this K quarter (the gate waves)
        if (p == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (r >= nr) break;
                const int64_t xr0 = row_token(g0 + r0 + r) * K32;
                float xs = 0.0f;
                for (int k = 32 * kb0 + lane; k < 32 * (kb0 + nkb); k += 64) xs += s_x[xr0 + k];
#pragma unroll
                for (int d = 32; d >= 1; d >>= 1) xs += __shfl_xor(xs, d, 64);
                if (lane == 0) s_xs[q][r] = xs;
            }
        }
        __syncthreads();
        if (tid < nr * 8) {
            const int r = tid >> 3, c = tid & 7;
            float x_sum = 0.0f, a0 = 0.0f, a1 = 0.0f;
#pragma unroll
            for (int j = 0; j < kGsQ; ++j) {
                x_sum += s_xs[j][r];
                a0 += s_red[0][j][r][c];
                a1 += s_red[1][j][r][c];
            }
            const float g = __fmul_rn(__fsub_rn(a0, __fmul_rn((float)(128 + zp[e * 3]), x_sum)), scale[e * 3]);
            const float uu = __fmul_rn(__fsub_rn(a1, __fmul_rn((float)(128 + zp[e * 3 + 1]), x_sum)),
                                       scale[e * 3 + 1]);
            const int64_t n = n0 + c;
            if (n < N) out[(g0 + r0 + r) * N + n] = __fmul_rn(hm_silu_t(g, s_exp2), uu);
        }
        __syncthreads();
    }
}

}  // namespace

#endif  // HM_GEMV_SLICE_H
