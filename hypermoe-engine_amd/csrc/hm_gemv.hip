// hm_gemv.hip -- the decode-size INT8 expert path: W8A32 GEMVs in FP32 that
// stream the selected experts' weights from HBM once.
//
// At decode (a few tokens, each expert sees one or two rows) the expert
// GEMMs are pure weight streams: 4.5 MiB of INT8 per selected expert and a
// handful of multiply-adds per byte.  The weights are read in their device
// layout of 32 x 32 tiles (hm_tile_offset): one wave-wide 16-byte load is a
// whole kilobyte tile, lane l holding column l % 32 and K bytes
// 16 (l / 32) .. +15 of it.  A lane's K positions depend only on the K tile,
// so a wave that walks the column tiles of one K tile keeps the matching 16
// activations per row in registers and reuses them for every column; the
// waves of a workgroup split K, and their partial sums meet in LDS in a
// fixed order.
//
// Arithmetic: the reference computes y = sum_k x_k * (float(q_k - zp) * s)
// in FP32 (CpuTensorBackend.cpp:173-186).  Here the dequantisation is
// factored: with u_k = q_k + 128 (the byte XOR 0x80, converted by
// v_cvt_f32_ubyteN),
//     y = s * (sum_k x_k u_k - (128 + zp) * sum_k x_k),
// summed in a different order; the result is within the north-star 1e-4 of
// the reference (rounding of FP32 sums of 2048 terms), not bit-identical to
// it.  SiLU(G)*U uses the same float operations as the other paths.
#include "hm_device.h"

namespace {

constexpr int kGvWaves = 4;                 // waves per workgroup (they split K)
constexpr int kGvThreads = 64 * kGvWaves;
constexpr int kGvCols = 8;                  // column tiles (32 columns) per workgroup
constexpr int kGvRows = 2;                  // activation rows per pass over the weights

typedef int v4i __attribute__((ext_vector_type(4)));

// The slot-th expert (ascending id) with a non-zero group; -1 if none.
// Every wave computes it redundantly from `counts` (E <= 1024); the loads
// of all 64-expert groups go out together.
__device__ int hm_active_expert(const int32_t* __restrict__ counts, int64_t experts, int slot) {
    const int lane = threadIdx.x & 63;
    constexpr int kGroups = 16;
    int cnt[kGroups];
#pragma unroll
    for (int b = 0; b < kGroups; ++b) {
        const int64_t e = (int64_t)b * 64 + lane;
        cnt[b] = e < experts ? counts[e] : 0;
    }
    int seen = 0;
#pragma unroll
    for (int b = 0; b < kGroups; ++b) {
        const unsigned long long m = __ballot(cnt[b] > 0);
        const int c = __popcll(m);
        if (slot < seen + c) {
            // position of the (slot - seen)-th set bit
            unsigned long long mm = m;
            for (int i = 0; i < slot - seen; ++i) mm &= mm - 1;
            return b * 64 + __ffsll((long long)mm) - 1;
        }
        seen += c;
    }
    return -1;
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

// The 16 activations of lane `lane` for K tile kb of row x (0 past K).
__device__ __forceinline__ void x_slice(const float* __restrict__ x, int64_t K, int kb, int lane,
                                        float (&v)[16]) {
    const int64_t k = 32 * (int64_t)kb + 16 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 t = k < K ? *reinterpret_cast<const float4*>(x + k + 4 * i)
                               : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
}

// ---------------------------------------------------------------------------
// GATEUP: z[g, n] = silu(x_g . Wg[n]) * (x_g . Wu[n]), x_g = hidden[perm_tokens[g]]
// DOWN:   y[g, n] = z_g . Wd[n]
// Workgroup: one active expert (blockIdx.y-th), kGvCols column tiles from
// blockIdx.x * kGvCols; wave w takes K tiles [w KT/4, (w+1) KT/4).
// ---------------------------------------------------------------------------
template <bool GATEUP>
__global__ __launch_bounds__(kGvThreads) void gemv_tiles_kernel(
    const float* __restrict__ x_src, const int32_t* __restrict__ perm_tokens, int64_t K,
    int64_t N, int64_t experts, const int8_t* __restrict__ packed, int64_t hidden,
    int64_t inter, const float* __restrict__ scale, const int32_t* __restrict__ zp,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    float* __restrict__ out) {
    constexpr int NP = GATEUP ? 2 : 1;  // projections
    __shared__ float s_red[kGvWaves][kGvRows][NP * kGvCols + 1][32];
    __shared__ unsigned long long s_exp2[32];
    if (GATEUP) hm_load_exp2_table(s_exp2);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int e = hm_active_expert(counts, experts, (int)blockIdx.y);
    __syncthreads();
    if (e < 0) return;
    const int64_t K32 = hm_pad32(K), KT = K32 / 32, NT = hm_pad32(N) / 32;
    const int cb0 = blockIdx.x * kGvCols;
    const int kb0 = (int)(wave * KT / kGvWaves), kb1 = (int)((wave + 1) * KT / kGvWaves);
    const int8_t* wbase[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p)
        wbase[p] = packed + hm_proj_offset(e, GATEUP ? p : 2, hidden, inter) + 16 * lane;
    const int64_t g0 = offsets[e];
    const int rows = counts[e];
    for (int r0 = 0; r0 < rows; r0 += kGvRows) {
        const int nr = min(kGvRows, rows - r0);
        const float* xr[kGvRows];
#pragma unroll
        for (int r = 0; r < kGvRows; ++r) {
            const int64_t g = g0 + r0 + min(r, nr - 1);
            xr[r] = x_src + (GATEUP ? (int64_t)perm_tokens[g] : g) * K;
        }
        float acc[kGvRows][NP * kGvCols], xs[kGvRows];
#pragma unroll
        for (int r = 0; r < kGvRows; ++r) {
            xs[r] = 0.0f;
#pragma unroll
            for (int c = 0; c < NP * kGvCols; ++c) acc[r][c] = 0.0f;
        }
        for (int kb = kb0; kb < kb1; ++kb) {
            // every tile of this K step first (one burst of loads)
            v4i w[NP * kGvCols];
#pragma unroll
            for (int p = 0; p < NP; ++p)
#pragma unroll
                for (int c = 0; c < kGvCols; ++c) {
                    const int cb = min(cb0 + c, (int)NT - 1);
                    w[p * kGvCols + c] = *reinterpret_cast<const v4i*>(wbase[p] + ((int64_t)cb * KT + kb) * 1024);
                }
            float xv[kGvRows][16];
#pragma unroll
            for (int r = 0; r < kGvRows; ++r) {
                x_slice(xr[r], K, kb, lane, xv[r]);
#pragma unroll
                for (int j = 0; j < 16; ++j) xs[r] += xv[r][j];
            }
#pragma unroll
            for (int c = 0; c < NP * kGvCols; ++c) {
                float f[16];
                tile_to_float(w[c], f);
#pragma unroll
                for (int r = 0; r < kGvRows; ++r)
#pragma unroll
                    for (int j = 0; j < 16; ++j) acc[r][c] = __builtin_fmaf(xv[r][j], f[j], acc[r][c]);
            }
        }
        // the two K halves of a column (lanes l, l + 32), then the waves in
        // order through LDS
#pragma unroll
        for (int r = 0; r < kGvRows; ++r) {
#pragma unroll
            for (int c = 0; c < NP * kGvCols; ++c) {
                const float v = acc[r][c] + __shfl_xor(acc[r][c], 32, 64);
                if (lane < 32) s_red[wave][r][c][lane] = v;
            }
            const float xv = xs[r] + __shfl_xor(xs[r], 32, 64);
            if (lane < 32) s_red[wave][r][NP * kGvCols][lane] = xv;
        }
        __syncthreads();
        // wave w finalises rows r = w (of the kGvRows) ... one row per wave
        for (int r = wave; r < nr; r += kGvWaves) {
            if (lane < 32) {
                // the activation sum (every lane of a wave holds its wave's
                // part), over the waves in order
                float x_sum = 0.0f;
                for (int w = 0; w < kGvWaves; ++w) x_sum += s_red[w][r][NP * kGvCols][0];
                const int64_t g = g0 + r0 + r;
#pragma unroll
                for (int c = 0; c < kGvCols; ++c) {
                    const int64_t n = 32 * (int64_t)(cb0 + c) + lane;
                    float t[NP];
#pragma unroll
                    for (int p = 0; p < NP; ++p) {
                        float a = 0.0f;
                        for (int w = 0; w < kGvWaves; ++w) a += s_red[w][r][p * kGvCols + c][lane];
                        const int pr = GATEUP ? p : 2;
                        t[p] = __fmul_rn(__fsub_rn(a, __fmul_rn((float)(128 + zp[e * 3 + pr]), x_sum)),
                                         scale[e * 3 + pr]);
                    }
                    if (cb0 + c < NT && n < N) {
                        if (GATEUP) out[g * N + n] = __fmul_rn(hm_silu_t(t[0], s_exp2), t[NP - 1]);
                        else out[g * N + n] = t[0];
                    }
                }
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Decode down projection fused with the combine, column-tile major: a
// workgroup owns one 32-column output tile for EVERY active expert (its 16
// waves take the experts in turn, each streaming the expert's down tiles of
// that column tile), keeps y[g, those columns] of every grouped row g in
// LDS, and then forms the tokens' outputs for its columns with hm_combine's
// arithmetic.  No workgroup needs another's results, so there is no
// device-wide synchronisation, and y goes to memory only when the caller
// asks for the expert outputs.  T <= 16, top_k <= 16, I <= 1024.
// ---------------------------------------------------------------------------
constexpr int kDcWaves = 16;
constexpr int kDcPairs = HM_GEMV_MAX_TOKENS * 16;
constexpr int kDcMaxKT = 32;  // I <= 1024

__global__ __launch_bounds__(64 * kDcWaves) void gemv_down_combine_kernel(
    const float* __restrict__ z, int64_t I, int64_t H, int64_t experts,
    const int8_t* __restrict__ packed, const float* __restrict__ scale,
    const int32_t* __restrict__ zp, const int32_t* __restrict__ counts,
    const int32_t* __restrict__ offsets, const uint32_t* __restrict__ ids,
    const int32_t* __restrict__ slots, const float* __restrict__ scores,
    const float* __restrict__ residual, int tokens, int top_k, float* __restrict__ y_out,
    float* __restrict__ out) {
    __shared__ float s_y[kDcPairs][32];
    __shared__ int s_cnt[1024], s_off[1024], s_act[1024];
    __shared__ int s_nact;
    __shared__ uint32_t s_ids[kDcPairs];
    __shared__ int s_row[HM_GEMV_MAX_TOKENS][16];
    __shared__ float s_w[HM_GEMV_MAX_TOKENS][16];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int cb = blockIdx.x;
    // every routing input the workgroup needs, in one round of loads
    const int pairs = tokens * top_k;
    for (int i = tid; i < experts; i += 64 * kDcWaves) {
        s_cnt[i] = counts[i];
        s_off[i] = offsets[i];
    }
    uint32_t my_id = 0;
    int my_slot = 0;
    float my_score = 0.0f;
    if (tid < pairs) {
        my_id = ids[tid];
        my_slot = slots[tid];
        my_score = scores[tid];
        s_ids[tid] = my_id;
    }
    for (int i = tid; i < HM_GEMV_MAX_TOKENS * 16; i += 64 * kDcWaves) {
        (&s_row[0][0])[i] = 0;  // (ranks collide only after a routing failure)
        (&s_w[0][0])[i] = 0.0f;
    }
    __syncthreads();
    // the active experts, ascending (wave 0 compacts the counts); the pairs'
    // ranks by expert id within their token
    if (wave == 0) {
        int seen = 0;
        for (int64_t base = 0; base < experts; base += 64) {
            const int64_t e = base + lane;
            const bool nz = e < experts && s_cnt[e] > 0;
            const unsigned long long m = __ballot(nz);
            if (nz) s_act[seen + __popcll(m & ((1ull << lane) - 1))] = (int)e;
            seen += __popcll(m);
        }
        if (lane == 0) s_nact = seen;
    }
    if (tid < pairs) {
        const int t = tid / top_k;
        int rank = 0;
        for (int q = 0; q < top_k; ++q) rank += s_ids[t * top_k + q] < my_id;
        s_row[t][rank & 15] = my_slot;
        s_w[t][rank & 15] = my_score;
    }
    __syncthreads();
    const int nact = s_nact;
    const int64_t KT = hm_pad32(I) / 32;
    for (int a = wave; a < nact; a += kDcWaves) {
        const int e = s_act[a];
        const int8_t* wt = packed + hm_proj_offset(e, 2, H, I) + (int64_t)cb * KT * 1024 + 16 * lane;
        // the expert's whole column tile (K <= 1024: at most 32 tiles)
        v4i w[kDcMaxKT];
#pragma unroll
        for (int kb = 0; kb < kDcMaxKT; ++kb)
            if (kb < KT) w[kb] = *reinterpret_cast<const v4i*>(wt + (int64_t)kb * 1024);
        const int64_t g0 = s_off[e];
        const int rows = s_cnt[e];
        const float sc = scale[e * 3 + 2];
        const float zc = (float)(128 + zp[e * 3 + 2]);
        for (int r = 0; r < rows; ++r) {
            const float* xr = z + (g0 + r) * I;
            float acc = 0.0f, xs = 0.0f;
#pragma unroll
            for (int kb = 0; kb < kDcMaxKT; ++kb) {
                if (kb < KT) {
                    float xv[16], f[16];
                    x_slice(xr, I, kb, lane, xv);
                    tile_to_float(w[kb], f);
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        acc = __builtin_fmaf(xv[j], f[j], acc);
                        xs += xv[j];
                    }
                }
            }
            acc += __shfl_xor(acc, 32, 64);
            // the activation sum: lanes l and l + 32 hold the sums of the two
            // K halves (the same in every column)
            const float xt = xs + __shfl_xor(xs, 32, 64);
            const float y = __fmul_rn(__fsub_rn(acc, __fmul_rn(zc, xt)), sc);
            const int64_t n = 32 * (int64_t)cb + lane;
            if (lane < 32) {
                s_y[(g0 + r) & (kDcPairs - 1)][lane] = y;
                if (y_out && n < H) y_out[(g0 + r) * H + n] = y;
            }
        }
    }
    // the combine of hm_combine (MoERuntime.cpp:308-325) for these columns
    __syncthreads();
    for (int i = tid; i < tokens * 32; i += 64 * kDcWaves) {
        const int t = i / 32, c = i % 32;
        const int64_t n = 32 * (int64_t)cb + c;
        if (n >= H) continue;
        float acc = 0.0f;
        for (int r = 0; r < top_k; ++r)
            acc = __fadd_rn(acc, __fmul_rn(s_w[t][r], s_y[s_row[t][r] & (kDcPairs - 1)][c]));
        if (residual) acc = __fadd_rn(residual[t * H + n], acc);
        out[t * H + n] = acc;
    }
}

template <bool GATEUP>
int launch_gemv(const float* x_src, const int32_t* perm_tokens, int64_t K, int64_t N,
                const hm_layer* L, const int32_t* counts, const int32_t* offsets, int64_t slots,
                float* out, hipStream_t s) {
    const int64_t nt = hm_pad32(N) / 32;
    const dim3 grid((unsigned)((nt + kGvCols - 1) / kGvCols), (unsigned)slots);
    // (the timer, when armed, brackets the gate/up launch)
    HM_STAGE_LAUNCH(true, true, (gemv_tiles_kernel<GATEUP>), grid, dim3(kGvThreads), 0, s, x_src,
                    perm_tokens, K, N, L->experts, static_cast<const int8_t*>(L->packed),
                    L->hidden, L->intermediate, L->scale, L->zero_point, counts, offsets, out);
    HM_LAUNCHED();
    return HM_OK;
}

}  // namespace

// Shapes the GEMV kernels take: H, I multiples of 16 (whole float4
// activation slices) up to 65536.
bool hm_gemv_shape_ok(int64_t H, int64_t I) {
    return H >= 16 && I >= 16 && H % 16 == 0 && I % 16 == 0 && H <= 65536 && I <= 65536;
}

// z[g, n] = silu(x_g . Wg[n]) * (x_g . Wu[n]) for every grouped row g, with
// x_g = hidden[perm_tokens[g]]; `pairs` = T*k bounds the active experts.
int hm_launch_gateup_gemv(const hm_layer* L, const float* hidden, const int32_t* counts,
                          const int32_t* offsets, const int32_t* perm_tokens, int64_t pairs,
                          float* z, hipStream_t s) {
    if (L->experts > 1024) return HM_ERR_UNSUPPORTED;
    const int64_t slots = pairs < L->experts ? pairs : L->experts;
    return launch_gemv<true>(hidden, perm_tokens, L->hidden, L->intermediate, L, counts, offsets,
                             slots, z, s);
}

// The decode down projection fused with the combine (T <= 16, top_k <= 16,
// I <= 1024); y_out (optional) receives the expert outputs.
bool hm_gemv_combine_ok(int64_t tokens, int32_t top_k, int64_t H, int64_t I) {
    return tokens <= HM_GEMV_MAX_TOKENS && top_k <= 16 && I <= 32 * kDcMaxKT && I % 16 == 0 &&
           H % 16 == 0;
}

int hm_launch_down_combine_gemv(const hm_layer* L, const float* z, const int32_t* counts,
                                const int32_t* offsets, const uint32_t* ids,
                                const int32_t* slots, const float* scores,
                                const float* residual, int64_t tokens, int32_t top_k,
                                float* y_out, float* out, hipStream_t s) {
    if (!hm_gemv_combine_ok(tokens, top_k, L->hidden, L->intermediate) || L->experts > 1024)
        return HM_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(gemv_down_combine_kernel, dim3((unsigned)(hm_pad32(L->hidden) / 32)),
                       dim3(64 * kDcWaves), 0, s, z, L->intermediate, L->hidden, L->experts,
                       static_cast<const int8_t*>(L->packed), L->scale, L->zero_point, counts,
                       offsets, ids, slots, scores, residual, (int)tokens, top_k, y_out, out);
    HM_LAUNCHED();
    return HM_OK;
}

// y[g, n] = z_g . Wd[n] for every grouped row g.
int hm_launch_down_gemv(const hm_layer* L, const float* z, const int32_t* counts,
                        const int32_t* offsets, int64_t pairs, float* y, hipStream_t s) {
    if (L->experts > 1024) return HM_ERR_UNSUPPORTED;
    const int64_t slots = pairs < L->experts ? pairs : L->experts;
    return launch_gemv<false>(z, nullptr, L->intermediate, L->hidden, L, counts, offsets, slots,
                              y, s);
}
