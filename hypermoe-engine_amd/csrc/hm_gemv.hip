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

constexpr int kGvWaves = 8;                 // waves per workgroup
constexpr int kGvThreads = 64 * kGvWaves;
constexpr int kGvRows = 4;                  // activation rows per pass (weights stay in registers)
constexpr int kGvMaxTiles = 16;             // K tiles per wave: K <= 32 * 16 * (waves per projection)

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

// ---------------------------------------------------------------------------
// GATEUP: z[g, n] = silu(x_g . Wg[n]) * (x_g . Wu[n]), x_g = hidden[perm_tokens[g]]
// DOWN:   y[g, n] = z_g . Wd[n]
// Workgroup: one active expert (the blockIdx.y-th) x CT 32-column tiles
// (from CT * blockIdx.x).  The waves split into (projection, column tile,
// K range): NP * CT * NQ = 8; each loads all its weight tiles first (one
// burst, held in registers) and then streams the expert's rows past them,
// kGvRows at a time, from an LDS copy of the rows.  Partial sums meet in LDS
// in a fixed order (the two K halves of a tile, then the K ranges in
// ascending order).  Dynamic LDS: kGvRows * K32 floats.
// ---------------------------------------------------------------------------
template <bool GATEUP, int CT>
__global__ __launch_bounds__(kGvThreads) void gemv_kernel(
    const float* __restrict__ x_src, const int32_t* __restrict__ perm_tokens, int64_t K,
    int64_t N, int64_t experts, const int8_t* __restrict__ packed, int64_t hidden,
    int64_t inter, const float* __restrict__ scale, const int32_t* __restrict__ zp,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    float* __restrict__ out) {
    constexpr int NP = GATEUP ? 2 : 1;           // projections
    constexpr int NQ = kGvWaves / (NP * CT);     // K ranges per (projection, column tile)
    static_assert(NQ >= 1 && NP * CT * NQ == kGvWaves, "wave split");
    extern __shared__ __attribute__((aligned(16))) float s_x[];      // [kGvRows][K32]
    __shared__ float s_red[NP][CT][NQ][kGvRows][32];
    __shared__ float s_xs[NQ][kGvRows];
    __shared__ unsigned long long s_exp2[32];
    if (GATEUP) hm_load_exp2_table(s_exp2);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int p = wave / (CT * NQ), c = (wave / NQ) % CT, q = wave % NQ;
    const int e = hm_active_expert(counts, experts, (int)blockIdx.y);
    if (e < 0) return;  // uniform: every wave computes the same e
    const int64_t K32 = hm_pad32(K), KT = K32 / 32;
    const int64_t NT = hm_pad32(N) / 32;
    const int cb = min((int)(CT * blockIdx.x) + c, (int)NT - 1);  // past the last tile: repeats it
    const int kb0 = (int)(q * KT / NQ), nkb = (int)((q + 1) * KT / NQ) - kb0;
    // the wave's weight tiles, all loads in flight together
    const int8_t* wt = packed + hm_proj_offset(e, GATEUP ? p : 2, hidden, inter) +
                       ((int64_t)cb * KT + kb0) * 1024 + 16 * lane;
    v4i w[kGvMaxTiles];
#pragma unroll
    for (int t = 0; t < kGvMaxTiles; ++t)
        if (t < nkb) w[t] = *reinterpret_cast<const v4i*>(wt + (int64_t)t * 1024);
    const int64_t g0 = offsets[e];
    const int rows = counts[e];
    for (int r0 = 0; r0 < rows; r0 += kGvRows) {
        const int nr = min(kGvRows, rows - r0);
        // the rows into LDS (zero past K: the padded K tiles hold zeros too)
        const int64_t k4 = K32 / 4;
        for (int64_t i = tid; i < (int64_t)nr * k4; i += kGvThreads) {
            const int r = (int)(i / k4);
            const int64_t k = 4 * (i % k4);
            const int64_t g = g0 + r0 + r;
            const float* xr = x_src + (GATEUP ? (int64_t)perm_tokens[g] : g) * K;
            const float4 v = k < K ? *reinterpret_cast<const float4*>(xr + k) : make_float4(0.f, 0.f, 0.f, 0.f);
            *reinterpret_cast<float4*>(&s_x[r * K32 + k]) = v;
        }
        __syncthreads();
        float acc[kGvRows], xs[kGvRows];
#pragma unroll
        for (int r = 0; r < kGvRows; ++r) acc[r] = xs[r] = 0.0f;
#pragma unroll
        for (int t = 0; t < kGvMaxTiles; ++t) {
            if (t < nkb) {
                float f[16];
                tile_to_float(w[t], f);
                const int64_t k = 32 * (int64_t)(kb0 + t) + 16 * (lane >> 5);
#pragma unroll
                for (int r = 0; r < kGvRows; ++r) {
                    if (r < nr) {
                        const float4* xv = reinterpret_cast<const float4*>(&s_x[r * K32 + k]);
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float4 v = xv[i];
                            acc[r] = __builtin_fmaf(v.x, f[4 * i], acc[r]);
                            acc[r] = __builtin_fmaf(v.y, f[4 * i + 1], acc[r]);
                            acc[r] = __builtin_fmaf(v.z, f[4 * i + 2], acc[r]);
                            acc[r] = __builtin_fmaf(v.w, f[4 * i + 3], acc[r]);
                            xs[r] += (v.x + v.y) + (v.z + v.w);
                        }
                    }
                }
            }
        }
        // the two K halves of each column (lanes l, l + 32), then the waves
#pragma unroll
        for (int r = 0; r < kGvRows; ++r) {
            const float a = acc[r] + __shfl_xor(acc[r], 32, 64);
            const float x = xs[r] + __shfl_xor(xs[r], 32, 64);
            if (lane < 32) s_red[p][c][q][r][lane] = a;
            if (p == 0 && c == 0 && lane == 0) s_xs[q][r] = x;
        }
        __syncthreads();
        // one half-wave per (row, column tile) finishes its 32 columns
        for (int u = tid / 32; u < nr * CT; u += 2 * kGvWaves) {
            const int r = u / CT, cc = u % CT, col = tid & 31;
            float x_sum = 0.0f;
#pragma unroll
            for (int j = 0; j < NQ; ++j) x_sum += s_xs[j][r];
            float v[NP];
#pragma unroll
            for (int pp = 0; pp < NP; ++pp) {
                float a = 0.0f;
#pragma unroll
                for (int j = 0; j < NQ; ++j) a += s_red[pp][cc][j][r][col];
                const int prr = GATEUP ? pp : 2;
                v[pp] = __fmul_rn(__fsub_rn(a, __fmul_rn((float)(128 + zp[e * 3 + prr]), x_sum)),
                                  scale[e * 3 + prr]);
            }
            const int64_t tile = (int64_t)CT * blockIdx.x + cc;
            const int64_t n = 32 * tile + col;
            const int64_t g = g0 + r0 + r;
            if (tile < NT && n < N) {
                if (GATEUP) out[g * N + n] = __fmul_rn(hm_silu_t(v[0], s_exp2), v[NP - 1]);
                else out[g * N + n] = v[0];
            }
        }
        __syncthreads();
    }
}

template <bool GATEUP, int CT>
int launch_gemv(const float* x_src, const int32_t* perm_tokens, int64_t K, int64_t N,
                const hm_layer* L, const int32_t* counts, const int32_t* offsets, int64_t slots,
                float* out, hipStream_t s) {
    constexpr int NQ = kGvWaves / ((GATEUP ? 2 : 1) * CT);
    const int64_t nt = hm_pad32(N) / 32, kt = hm_pad32(K) / 32;
    // every wave's K range within its register tiles
    if ((kt + NQ - 1) / NQ > kGvMaxTiles) return HM_ERR_UNSUPPORTED;
    const dim3 grid((unsigned)((nt + CT - 1) / CT), (unsigned)slots);
    const size_t lds = (size_t)kGvRows * hm_pad32(K) * sizeof(float);
    // (the timer, when armed, brackets the gate/up launch)
    HM_STAGE_LAUNCH(true, true, (gemv_kernel<GATEUP, CT>), grid, dim3(kGvThreads), lds, s, x_src,
                    perm_tokens, K, N, L->experts, static_cast<const int8_t*>(L->packed),
                    L->hidden, L->intermediate, L->scale, L->zero_point, counts, offsets, out);
    HM_LAUNCHED();
    return HM_OK;
}

}  // namespace

// Shapes the GEMV kernels take: H, I multiples of 16 (whole float4
// activation slices); K (H for gate/up, I for down) within the waves'
// register tiles (kGvMaxTiles K tiles per wave) and the LDS row copies.
bool hm_gemv_shape_ok(int64_t H, int64_t I) {
    const int64_t kmax_gu = 32 * kGvMaxTiles * (kGvWaves / 2), kmax_dn = 32 * kGvMaxTiles * kGvWaves;
    return H >= 16 && I >= 16 && H % 16 == 0 && I % 16 == 0 && H <= kmax_gu && I <= kmax_dn &&
           H <= 4096 && I <= 4096;
}

// z[g, n] = silu(x_g . Wg[n]) * (x_g . Wu[n]) for every grouped row g, with
// x_g = hidden[perm_tokens[g]]; `pairs` = T*k bounds the active experts.
int hm_launch_gateup_gemv(const hm_layer* L, const float* hidden, const int32_t* counts,
                          const int32_t* offsets, const int32_t* perm_tokens, int64_t pairs,
                          float* z, hipStream_t s) {
    if (L->experts > 1024) return HM_ERR_UNSUPPORTED;
    const int64_t slots = pairs < L->experts ? pairs : L->experts;
    return launch_gemv<true, 1>(hidden, perm_tokens, L->hidden, L->intermediate, L, counts,
                                offsets, slots, z, s);
}

// y[g, n] = z_g . Wd[n] for every grouped row g.
int hm_launch_down_gemv(const hm_layer* L, const float* z, const int32_t* counts,
                        const int32_t* offsets, int64_t pairs, float* y, hipStream_t s) {
    if (L->experts > 1024) return HM_ERR_UNSUPPORTED;
    const int64_t slots = pairs < L->experts ? pairs : L->experts;
    // few experts: one column tile per workgroup (more workgroups in
    // flight); many: four (a workgroup's setup spread over four times the
    // weights)
    if (slots >= 32 && hm_pad32(L->intermediate) / 32 <= 2 * kGvMaxTiles)
        return launch_gemv<false, 4>(z, nullptr, L->intermediate, L->hidden, L, counts, offsets,
                                     slots, y, s);
    return launch_gemv<false, 1>(z, nullptr, L->intermediate, L->hidden, L, counts, offsets, slots,
                                 y, s);
}
