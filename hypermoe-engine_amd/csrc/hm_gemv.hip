// hm_gemv.hip -- the decode-size INT8 expert path: W8A32 GEMVs in FP32 that
// stream the selected experts' weights from HBM once.
//
// At decode (a few tokens, each expert sees one or two rows) the expert
// GEMMs are pure weight streams: 4.5 MiB of INT8 per selected expert and a
// handful of multiply-adds per byte.  These kernels split K across the 64
// lanes of a wave (each lane owns fixed 16-byte slices of every weight row
// and the matching activation slices), stream each weight row once from HBM
// with coalesced 16-byte loads, and reduce the per-lane partial dot products
// of all of a wave's outputs across the wave in one butterfly.
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
#include "hm_lds_dma.h"

namespace {

constexpr int kGemvThreads = 256;
// Weight rows per wave (RW): 4, or 8 for gate/up when the batch selects many
// experts (more bytes in flight per wave; at one token the extra columns per
// workgroup only lengthen each wave's critical path).
constexpr int kRowsPerWave = 4;

// The slot-th expert (ascending id) with a non-zero group; -1 if none.
// Every wave computes it redundantly from `counts` (E <= 1024); the loads
// of all 64-expert groups go out together (two groups at E = 128).
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

// The same for E <= 256 with every count load issued at once (one round
// trip instead of one per 64-expert group).
__device__ int hm_active_expert_256(const int32_t* __restrict__ counts, int64_t experts,
                                    int slot) {
    const int lane = threadIdx.x & 63;
    int cnt[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const int64_t e = (int64_t)b * 64 + lane;
        const int c = counts[e < experts ? e : experts - 1];
        cnt[b] = e < experts ? c : 0;
    }
    int seen = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const unsigned long long m = __ballot(cnt[b] > 0);
        const int c = __popcll(m);
        if (slot < seen + c) {
            unsigned long long mm = m;
            for (int i = 0; i < slot - seen; ++i) mm &= mm - 1;
            return b * 64 + __ffsll((long long)mm) - 1;
        }
        seen += c;
    }
    return -1;
}

// Butterfly reduction of N (power of two, <= 64) values across the wave.
// Afterwards lane l holds the full sum of value index (l >> (6 - log2 N)),
// i.e. value i sits in lanes [i*64/N, (i+1)*64/N).
template <int N>
__device__ __forceinline__ float wave_reduce_many(float (&v)[N]) {
    const int lane = threadIdx.x & 63;
    int n = N;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        if (n > 1) {
            const bool upper = (lane & m) != 0;
#pragma unroll
            for (int i = 0; i < N / 2; ++i) {
                if (i < n / 2) {
                    const float send = upper ? v[i] : v[i + n / 2];
                    const float keep = upper ? v[i + n / 2] : v[i];
                    v[i] = keep + __shfl_xor(send, m, 64);
                }
            }
            n >>= 1;
        } else {
            v[0] += __shfl_xor(v[0], m, 64);
        }
    }
    return v[0];
}

// 4 unsigned bytes of a dword (after XOR 0x80) -> 4 floats
__device__ __forceinline__ void bytes_to_float(uint32_t d, float* f) {
    const uint32_t u = d ^ 0x80808080u;   // v_cvt_f32_ubyte0..3 below
    f[0] = (float)(u & 0xffu);
    f[1] = (float)((u >> 8) & 0xffu);
    f[2] = (float)((u >> 16) & 0xffu);
    f[3] = (float)(u >> 24);
}

// Lane slices of a K-long row (K % 16 == 0, K <= 1024*P): piece p of lane
// l is the 16 bytes at k = 1024 p + 16 l, present when that is below K.
//
// A wave owns RW weight rows.  Each lane loads its own 16-byte
// slices of them straight into registers (the lane later uses only the
// bytes it loaded, so nothing is shared through LDS and nothing waits on
// another wave); every activation row of the expert's group then meets
// them, the rows' partial sums are reduced together, and the weights are
// read from HBM once whatever the group size.
//
// GATEUP: rows j < RW/2 are gate rows n0+j, the others the up rows of the
// same n; the inputs are hidden[perm_tokens[g]]; the output z[g, n] =
// silu(g)*u.
// DOWN: rows j are down rows n0+j; the inputs are z[g, :]; output y[g, n].
template <int P, bool GATEUP, int RW>
__device__ __forceinline__ void gemv_body(
    const float* __restrict__ x_src, const int32_t* __restrict__ perm_tokens, int64_t K,
    int64_t N, const int8_t* __restrict__ packed, int64_t hidden, int64_t inter,
    const float* __restrict__ scale, const int32_t* __restrict__ zp,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    float* __restrict__ out, const unsigned long long* s_exp2, int e, int lane,
    int wave) {
    constexpr int kWaves = kGemvThreads / 64;
    const int8_t* ebase = packed + (int64_t)e * 3 * hidden * inter;
    constexpr int kNPW = RW / 2;  // gate/up: output columns per wave
    const int64_t n0 = GATEUP ? ((int64_t)blockIdx.x * kWaves + wave) * kNPW
                              : ((int64_t)blockIdx.x * kWaves + wave) * RW;
    const int64_t g0 = offsets[e];
    const int rows = counts[e];
    // weights -> registers: lane l's own 16-byte slices of every row (all
    // loads go out before the activations')
    uint4 wreg[RW][P];
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        const int proj = GATEUP ? j / kNPW : 2;
        const int64_t n = GATEUP ? n0 + j % kNPW : n0 + j;
        const int8_t* row = ebase + proj * hidden * inter + n * K;
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int64_t k = 1024 * p + 16 * lane;
            wreg[j][p] = k < K ? *reinterpret_cast<const uint4*>(row + k) : make_uint4(0, 0, 0, 0);
        }
    }
    // each row's activations are loaded before the wait: the first row's
    // stream in beside the weights
    for (int r = 0; r < rows; ++r) {
        const int64_t src = GATEUP ? (int64_t)perm_tokens[g0 + r] : g0 + r;
        const float* xr = x_src + src * K;
        float x[P][16];
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int64_t k = 1024 * p + 16 * lane;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 v = k < K ? *reinterpret_cast<const float4*>(xr + k + 4 * i)
                                       : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                x[p][4 * i] = v.x; x[p][4 * i + 1] = v.y;
                x[p][4 * i + 2] = v.z; x[p][4 * i + 3] = v.w;
            }
        }
        float xs = 0.0f;
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
            for (int i = 0; i < 16; ++i) xs += x[p][i];
        float xv[1] = {xs};
        const float xsum = wave_reduce_many<1>(xv);
        // the partial dot products of all RW weight rows, then one
        // reduction for all of them (row j's sum lands in lanes 16j .. 16j+15)
        float a[RW];
#pragma unroll
        for (int j = 0; j < RW; ++j) {
            a[j] = 0.0f;
#pragma unroll
            for (int p = 0; p < P; ++p) {
                // lanes without a piece hold zero weights; x is 0 there too
                const uint32_t d[4] = {wreg[j][p].x, wreg[j][p].y, wreg[j][p].z, wreg[j][p].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    // converted per row (hoisted out of the row loop, every
                    // weight row's floats would stay live)
                    uint32_t dq = d[q];
                    asm volatile("" : "+v"(dq));
                    float f[4];
                    bytes_to_float(dq, f);
#pragma unroll
                    for (int b = 0; b < 4; ++b) a[j] = __builtin_fmaf(x[p][4 * q + b], f[b], a[j]);
                }
            }
        }
        const float tot = wave_reduce_many<RW>(a);
        // lane 16j holds row j's sum; each output lane gathers its rows
        constexpr int kSpan = HM_WAVE / RW;
        if (GATEUP) {
            // lanes 0 .. kNPW-1: output o = lane from gate row o and up row kNPW+o
            const int o = lane < kNPW ? lane : 0;
            const float tg = __shfl(tot, kSpan * o, HM_WAVE);
            const float tu = __shfl(tot, kSpan * (kNPW + o), HM_WAVE);
            const float vg = __fmul_rn(__fsub_rn(tg, __fmul_rn((float)(128 + zp[e * 3 + 0]), xsum)),
                                       scale[e * 3 + 0]);
            const float vu = __fmul_rn(__fsub_rn(tu, __fmul_rn((float)(128 + zp[e * 3 + 1]), xsum)),
                                       scale[e * 3 + 1]);
            if (lane < kNPW) out[(g0 + r) * N + n0 + o] = __fmul_rn(hm_silu_t(vg, s_exp2), vu);
        } else {
            const float v = __fmul_rn(__fsub_rn(tot, __fmul_rn((float)(128 + zp[e * 3 + 2]), xsum)),
                                      scale[e * 3 + 2]);
            if (lane % kSpan == 0) out[(g0 + r) * N + n0 + lane / kSpan] = v;
        }
    }
}

template <int P, bool GATEUP, int RW>
__global__ __launch_bounds__(kGemvThreads) void gemv_w8_kernel(
    const float* __restrict__ x_src, const int32_t* __restrict__ perm_tokens, int64_t K,
    int64_t N, int64_t experts, const int8_t* __restrict__ packed, int64_t hidden,
    int64_t inter, const float* __restrict__ scale, const int32_t* __restrict__ zp,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    float* __restrict__ out) {
    constexpr int kWaves = kGemvThreads / 64;
    __shared__ unsigned long long s_exp2[32];
    if (GATEUP) hm_load_exp2_table(s_exp2);
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int e = experts <= 256 ? hm_active_expert_256(counts, experts, (int)blockIdx.y)
                                 : hm_active_expert(counts, experts, (int)blockIdx.y);
    if (e < 0) return;
    gemv_body<P, GATEUP, RW>(x_src, perm_tokens, K, N, packed, hidden, inter, scale, zp, counts,
                         offsets, out, s_exp2, e, lane, wave);
}

template <int P, bool GATEUP, int RW>
int launch_gemv(const float* x_src, const int32_t* perm_tokens, int64_t K, int64_t N,
                const hm_layer* L, const int32_t* counts, const int32_t* offsets, int64_t slots,
                float* out, hipStream_t s) {
    const int64_t per_wg = (kGemvThreads / 64) * (GATEUP ? RW / 2 : RW);
    const dim3 grid((unsigned)(N / per_wg), (unsigned)slots);
    // (the timer, when armed, brackets the gate/up launch)
    HM_STAGE_LAUNCH(true, true, (gemv_w8_kernel<P, GATEUP, RW>), grid, dim3(kGemvThreads), 0, s,
                    x_src, perm_tokens, K, N, L->experts, static_cast<const int8_t*>(L->packed),
                    L->hidden, L->intermediate, L->scale, L->zero_point, counts, offsets, out);
    HM_LAUNCHED();
    return HM_OK;
}

template <bool GATEUP>
int dispatch_gemv(int64_t K, const float* x_src, const int32_t* perm_tokens, int64_t N,
                  const hm_layer* L, const int32_t* counts, const int32_t* offsets,
                  int64_t slots, float* out, hipStream_t s) {
    // gate/up of a batch with many selected experts: 8 weight rows per wave
    // (N must then be a multiple of the 16-column workgroup)
    if constexpr (GATEUP) {
        if (slots >= 64 && N % 16 == 0) {
            if (K <= 1024) return launch_gemv<1, true, 8>(x_src, perm_tokens, K, N, L, counts, offsets, slots, out, s);
            if (K <= 2048) return launch_gemv<2, true, 8>(x_src, perm_tokens, K, N, L, counts, offsets, slots, out, s);
        }
    }
    if (K <= 1024) return launch_gemv<1, GATEUP, kRowsPerWave>(x_src, perm_tokens, K, N, L, counts, offsets, slots, out, s);
    if (K <= 2048) return launch_gemv<2, GATEUP, kRowsPerWave>(x_src, perm_tokens, K, N, L, counts, offsets, slots, out, s);
    return HM_ERR_UNSUPPORTED;
}

// ---------------------------------------------------------------------------
// Decode down projection fused with the combine, column-block major: a
// workgroup owns kDcCols output columns n0 .. n0+kDcCols-1 for EVERY active
// expert (its 16 waves take the experts in turn, each streaming the
// expert's kDcCols down rows into its LDS slot), keeps y[g, n0 ..] of every
// grouped row g in LDS, and then forms the tokens' outputs for its columns
// with hm_combine's arithmetic.  No workgroup needs another's results, so
// there is no device-wide synchronisation, and y goes to memory only when
// the caller asks for the expert outputs.  Each y uses gemv_body's DOWN
// lane slices; the 8 columns' partial sums are reduced across the wave
// together (one butterfly for all of them, not one per column), so y
// agrees with the two-kernel path to rounding.  T <= 16, top_k <= 16,
// I <= 1024.
// ---------------------------------------------------------------------------
constexpr int kDcCols = 8;
constexpr int kDcWaves = 16;
constexpr int kDcPairs = HM_GEMV_MAX_TOKENS * 16;

__global__ __launch_bounds__(64 * kDcWaves) void gemv_down_combine_kernel(
    const float* __restrict__ z, int64_t I, int64_t H, int64_t experts,
    const int8_t* __restrict__ packed, const float* __restrict__ scale,
    const int32_t* __restrict__ zp, const int32_t* __restrict__ counts,
    const int32_t* __restrict__ offsets, const uint32_t* __restrict__ ids,
    const int32_t* __restrict__ slots, const float* __restrict__ scores,
    const float* __restrict__ residual, int tokens, int top_k, float* __restrict__ y_out,
    float* __restrict__ out) {
    __shared__ __attribute__((aligned(1024))) int8_t wl[kDcWaves][kDcCols * 1024];
    __shared__ float s_y[kDcPairs][kDcCols];
    __shared__ int s_cnt[1024], s_off[1024], s_act[1024];
    __shared__ int s_nact;
    __shared__ uint32_t s_ids[kDcPairs];
    __shared__ int s_row[HM_GEMV_MAX_TOKENS][16];
    __shared__ float s_w[HM_GEMV_MAX_TOKENS][16];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t n0 = (int64_t)blockIdx.x * kDcCols;
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
    const int64_t K = I;
    int8_t* lds = wl[wave];
    for (int a = wave; a < nact; a += kDcWaves) {
        const int e = s_act[a];
        const int8_t* wrows = packed + (int64_t)e * 3 * H * I + 2 * H * I + n0 * K;
        const int64_t k = 16 * lane;
        __builtin_amdgcn_wave_barrier();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slot's last reads are done
        if (k < K) {
#pragma unroll
            for (int j = 0; j < kDcCols; ++j) dma16(wrows + j * K + k, lds + j * 1024);
        }
        const int64_t g0 = s_off[e];
        const int rows = s_cnt[e];
        const float sc = scale[e * 3 + 2];
        const float zc = (float)(128 + zp[e * 3 + 2]);
        wait_vmcnt<0>();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        for (int r = 0; r < rows; ++r) {
            const float* xr = z + (g0 + r) * K;
            float x[16];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 v = k < K ? *reinterpret_cast<const float4*>(xr + k + 4 * i)
                                       : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
            }
            float xs = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) xs += x[i];
            float xv[1] = {xs};
            const float xsum = wave_reduce_many<1>(xv);
            // the kDcCols partial dot products of this lane, then one
            // reduction for all of them (column j ends up in lanes 8j .. 8j+7)
            float acc[kDcCols];
#pragma unroll
            for (int j = 0; j < kDcCols; ++j) {
                acc[j] = 0.0f;
                // lanes without a piece read their own unused slot; x is 0
                const uint4 wv = *reinterpret_cast<const uint4*>(lds + j * 1024 + 16 * lane);
                const uint32_t d[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    // converted per row (hoisted out of the row loop, the 8
                    // rows' 128 floats would spill)
                    uint32_t dq = d[q];
                    asm volatile("" : "+v"(dq));
                    float f[4];
                    bytes_to_float(dq, f);
#pragma unroll
                    for (int b = 0; b < 4; ++b) acc[j] = __builtin_fmaf(x[4 * q + b], f[b], acc[j]);
                }
            }
            const float tot = wave_reduce_many<kDcCols>(acc);
            const int jl = lane / (HM_WAVE / kDcCols);
            const float y = __fmul_rn(__fsub_rn(tot, __fmul_rn(zc, xsum)), sc);
            if (lane % (HM_WAVE / kDcCols) == 0) {
                s_y[(g0 + r) & (kDcPairs - 1)][jl] = y;
                if (y_out) y_out[(g0 + r) * H + n0 + jl] = y;
            }
        }
    }
    // the combine of hm_combine (MoERuntime.cpp:308-325) for these columns
    __syncthreads();
    for (int i = tid; i < tokens * kDcCols; i += 64 * kDcWaves) {
        const int t = i / kDcCols, c = i % kDcCols;
        float acc = 0.0f;
        for (int r = 0; r < top_k; ++r)
            acc = __fadd_rn(acc, __fmul_rn(s_w[t][r], s_y[s_row[t][r] & (kDcPairs - 1)][c]));
        const int64_t n = n0 + c;
        if (residual) acc = __fadd_rn(residual[t * H + n], acc);
        out[t * H + n] = acc;
    }
}

// Rows up to 2048 bytes keep a wave's 8 weight rows within 16 KB of LDS.
bool gemv_k_ok(int64_t K) { return K >= 16 && K % 16 == 0 && K <= 2048; }

}  // namespace

// Shapes the GEMV kernels take: H, I multiples of 16 up to 2048 (the
// tiles: 8 gate/up columns and 16 down rows per workgroup).
bool hm_gemv_shape_ok(int64_t H, int64_t I) {
    return gemv_k_ok(H) && gemv_k_ok(I) && I % 8 == 0 && H % 16 == 0;
}

// z[g, n] = silu(x_g . Wg[n]) * (x_g . Wu[n]) for every grouped row g, with
// x_g = hidden[perm_tokens[g]]; `pairs` = T*k bounds the active experts.
int hm_launch_gateup_gemv(const hm_layer* L, const float* hidden, const int32_t* counts,
                          const int32_t* offsets, const int32_t* perm_tokens, int64_t pairs,
                          float* z, hipStream_t s) {
    const int64_t slots = pairs < L->experts ? pairs : L->experts;
    return dispatch_gemv<true>(L->hidden, hidden, perm_tokens, L->intermediate, L, counts,
                               offsets, slots, z, s);
}

// The decode down projection fused with the combine (T <= 16, top_k <= 16,
// I <= 1024, H % 8 == 0); y_out (optional) receives the expert outputs.
bool hm_gemv_combine_ok(int64_t tokens, int32_t top_k, int64_t H, int64_t I) {
    return tokens <= HM_GEMV_MAX_TOKENS && top_k <= 16 && I <= 1024 && I % 16 == 0 &&
           H % kDcCols == 0;
}

int hm_launch_down_combine_gemv(const hm_layer* L, const float* z, const int32_t* counts,
                                const int32_t* offsets, const uint32_t* ids,
                                const int32_t* slots, const float* scores,
                                const float* residual, int64_t tokens, int32_t top_k,
                                float* y_out, float* out, hipStream_t s) {
    if (!hm_gemv_combine_ok(tokens, top_k, L->hidden, L->intermediate) || L->experts > 1024)
        return HM_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(gemv_down_combine_kernel, dim3((unsigned)(L->hidden / kDcCols)),
                       dim3(64 * kDcWaves), 0, s, z, L->intermediate, L->hidden, L->experts,
                       static_cast<const int8_t*>(L->packed), L->scale, L->zero_point, counts,
                       offsets, ids, slots, scores, residual, (int)tokens, top_k, y_out, out);
    HM_LAUNCHED();
    return HM_OK;
}

// y[g, n] = z_g . Wd[n] for every grouped row g.
int hm_launch_down_gemv(const hm_layer* L, const float* z, const int32_t* counts,
                        const int32_t* offsets, int64_t pairs, float* y, hipStream_t s) {
    const int64_t slots = pairs < L->experts ? pairs : L->experts;
    return dispatch_gemv<false>(L->intermediate, z, nullptr, L->hidden, L, counts, offsets,
                                slots, y, s);
}
