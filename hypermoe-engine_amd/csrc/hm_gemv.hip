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
#include "hm_gemv_slice.h"

namespace {

// The slot-th expert (ascending id) with a non-zero group; -1 if none
// (gemv_kernel's scan).
// Every wave computes it redundantly from `counts` (E <= 1024); the loads
// of all 64-expert groups go out together.
__device__ int hm_active_expert_scan(const int32_t* __restrict__ counts, int64_t experts, int slot) {
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
    const int e = hm_active_expert_scan(counts, experts, (int)blockIdx.y);
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
        // the rows' sums over this wave's K range, once per row (the waves
        // of projection 0, column tile 0), not in the weight loop below
        if (p == 0 && c == 0) {
            for (int r = 0; r < nr; ++r) {
                float xs = 0.0f;
                for (int64_t k = 32 * (int64_t)kb0 + lane; k < 32 * (int64_t)(kb0 + nkb); k += 64)
                    xs += s_x[r * K32 + k];
#pragma unroll
                for (int d = 32; d >= 1; d >>= 1) xs += __shfl_xor(xs, d, 64);
                if (lane == 0) s_xs[q][r] = xs;
            }
        }
        float acc[kGvRows];
#pragma unroll
        for (int r = 0; r < kGvRows; ++r) acc[r] = 0.0f;
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
                        }
                    }
                }
            }
        }
        // the two K halves of each column (lanes l, l + 32), then the waves
#pragma unroll
        for (int r = 0; r < kGvRows; ++r) {
            const float a = acc[r] + __shfl_xor(acc[r], 32, 64);
            if (lane < 32) s_red[p][c][q][r][lane] = a;
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


// ---------------------------------------------------------------------------
// FP32-weight experts at decode (A5' for a few tokens; CpuTensorBackend::
// matmul, CpuTensorBackend.cpp:87-131, on each expert's rows):
//   GATEUP: z[g, n] = silu(x_g . Wg[n]) * (x_g . Wu[n]),  x_g = hidden[perm_tokens[g]]
//   DOWN:   y[g, n] = z_g . Wd[n]
// FP32 projections are stored [N][K] (hm_pack_layer), so each output
// column's weights are one contiguous row of K floats.  Workgroup: one
// active expert (the blockIdx.y-th) x NC columns; wave w takes projection
// w / (8 / NP) and CW columns, and holds their rows in registers (lane l:
// floats 4 l + 256 j .. +3 of each, K / 256 <= MJ float4); the expert's
// rows are staged in LDS kGvRows at a time.  Each (row, column) sum: per
// lane in j order, then a fixed butterfly over the wave.  The sums' order
// differs from the reference's sequential one: within the FP32 path's
// 1e-3, as the matrix-core kernels.  SiLU and the product as
// Activation.cpp:44 then the multiply.
// ---------------------------------------------------------------------------
constexpr int kF32Mj = 8;      // float4 per lane per column: K <= 2048

template <bool GATEUP, int CW, int MJ>
__global__ __launch_bounds__(kGvThreads) void gemv_f32_kernel(
    const float* __restrict__ x_src, const int32_t* __restrict__ perm_tokens, int64_t K,
    int64_t N, int64_t experts, const float* __restrict__ packed, int64_t hidden,
    int64_t inter, const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    float* __restrict__ out) {
    constexpr int NP = GATEUP ? 2 : 1;
    constexpr int WPP = kGvWaves / NP;        // waves per projection
    constexpr int NC = WPP * CW;              // columns per workgroup
    extern __shared__ __attribute__((aligned(16))) float s_x[];  // [kGvRows][K]
    __shared__ float s_acc[NP][NC][kGvRows];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int p = wave / WPP, cw = wave % WPP;
    const int e = hm_active_expert_scan(counts, experts, (int)blockIdx.y);
    if (e < 0) return;  // uniform: every wave computes the same e
    const int nj = (int)(K / 256);
    const float* proj = packed + ((int64_t)e * 3 + (GATEUP ? p : 2)) * hidden * inter;
    const int64_t nb = (int64_t)NC * blockIdx.x + CW * cw;
    // the wave's column rows, all loads in flight together (columns past N
    // repeat the last one and are not stored)
    float4 w[CW][MJ];
#pragma unroll
    for (int c = 0; c < CW; ++c) {
        const float* wr = proj + min(nb + c, N - 1) * K + 4 * lane;
#pragma unroll
        for (int j = 0; j < MJ; ++j)
            if (j < nj) w[c][j] = *reinterpret_cast<const float4*>(wr + 256 * j);
    }
    const int64_t g0 = offsets[e];
    const int rows = counts[e];
    for (int r0 = 0; r0 < rows; r0 += kGvRows) {
        const int nr = min(kGvRows, rows - r0);
        const int64_t k4 = K / 4;
        for (int64_t i = tid; i < (int64_t)nr * k4; i += kGvThreads) {
            const int r = (int)(i / k4);
            const int64_t k = 4 * (i % k4);
            const int64_t g = g0 + r0 + r;
            const float* xr = x_src + (GATEUP ? (int64_t)perm_tokens[g] : g) * K;
            *reinterpret_cast<float4*>(&s_x[r * K + k]) = *reinterpret_cast<const float4*>(xr + k);
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < kGvRows; ++r) {
            if (r < nr) {
#pragma unroll
                for (int c = 0; c < CW; ++c) {
                    float acc = 0.0f;
#pragma unroll
                    for (int j = 0; j < MJ; ++j) {
                        if (j < nj) {
                            const float4 xv = *reinterpret_cast<const float4*>(&s_x[r * K + 4 * lane + 256 * j]);
                            acc = __builtin_fmaf(xv.x, w[c][j].x, acc);
                            acc = __builtin_fmaf(xv.y, w[c][j].y, acc);
                            acc = __builtin_fmaf(xv.z, w[c][j].z, acc);
                            acc = __builtin_fmaf(xv.w, w[c][j].w, acc);
                        }
                    }
#pragma unroll
                    for (int d = 32; d >= 1; d >>= 1) acc += __shfl_xor(acc, d, HM_WAVE);
                    if (lane == 0) s_acc[p][CW * cw + c][r] = acc;
                }
            }
        }
        __syncthreads();
        if (tid < nr * NC) {
            const int r = tid / NC, c = tid % NC;
            const int64_t n = (int64_t)NC * blockIdx.x + c;
            if (n < N) {
                const float v = GATEUP ? __fmul_rn(hm_silu(s_acc[0][c][r]), s_acc[NP - 1][c][r])
                                       : s_acc[0][c][r];
                out[(g0 + r0 + r) * N + n] = v;
            }
        }
        __syncthreads();
    }
}


template <int NG, int LJ>
__global__ __launch_bounds__(kGvThreads) void gateup_slice_kernel(
    const float* __restrict__ x_src, const int32_t* __restrict__ perm_tokens, int64_t K,
    int64_t N, int64_t experts, const int8_t* __restrict__ packed, const float* __restrict__ scale,
    const int32_t* __restrict__ zp, const int32_t* __restrict__ counts, int n_tokens,
    float* __restrict__ out) {
    gateup_slice_body<NG, LJ, false>(blockIdx.x, blockIdx.y, hm_slice_pre{-1, 0, 0, -1}, x_src,
                                     perm_tokens, K, N, experts, packed, scale, zp, counts,
                                     n_tokens, out);
}

// ---------------------------------------------------------------------------
// Decode down projection fused with the combine, for few (token, expert)
// pairs (P = T*k <= kDcPairs), with no workgroup waiting for another: the
// workgroup owns kDcCols = 8 output columns for every active expert (H/8
// workgroups, enough to keep every CU streaming) and forms the tokens'
// outputs for them itself.
//
// Eight columns of a tile are two 128-byte pieces of it (K halves 0 and 1:
// bytes 128 s .. +127 and 512 + 128 s .. +127 for slice s), so one
// wave-wide 16-byte load covers four K tiles: lane l takes tile l / 16, K
// half (l / 8) % 2, column l % 8.  The waves split (active expert, K range):
// with nact < 8 active experts 8 / nact waves share an expert's K, with
// nact >= 8 a wave takes experts wave and wave + 8 whole.  Each wave holds
// its expert's pieces in registers and runs the expert's z rows (staged in
// LDS) past them; the eight lanes of a column sum in a fixed tree, the waves
// of an expert in K order, and
//   y[g, n] = s (sum_k z_k u_k - (128 + zp) sum_k z_k),  u = q + 128,
// as in gemv_kernel.  The combine follows hm_combine's arithmetic (pairs by
// ascending expert id from 0, residual added last).  Every load that needs
// no routing result (z, the residual, counts) is issued first.
// ---------------------------------------------------------------------------
constexpr int kDcWaves = 8;
constexpr int kDcThreads = 64 * kDcWaves;
constexpr int kDcPairs = 16;                    // P = T * k
constexpr int kDcCols = 8;                      // output columns per workgroup
constexpr int kDcMaxTiles = 24;                 // K tiles of down: I <= 32 * 24
constexpr int kDcLoads = kDcMaxTiles / 4;       // wave loads per expert (four K tiles each)
constexpr int kDcZ = (kDcPairs * 32 * kDcMaxTiles / 4 + kDcThreads - 1) / kDcThreads;  // z float4 per thread

// NG: 64-expert groups (E <= 64 NG)
template <int NG>
__global__ __launch_bounds__(kDcThreads) void gemv_down_combine_kernel(
    const float* __restrict__ z, int64_t I, int64_t H, int64_t experts,
    const int8_t* __restrict__ packed, const float* __restrict__ scale,
    const int32_t* __restrict__ zp, const int32_t* __restrict__ counts,
    const uint32_t* __restrict__ ids, const int32_t* __restrict__ slots,
    const float* __restrict__ scores, const float* __restrict__ residual, int tokens,
    int top_k, float* __restrict__ y_out, float* __restrict__ out) {
    extern __shared__ __attribute__((aligned(16))) float s_z[];      // [P][I32]
    __shared__ float s_part[kDcWaves][2][kDcPairs][kDcCols];         // per wave, unit, row
    __shared__ float s_zs[kDcWaves][2][kDcPairs];                    // the rows' z sums
    __shared__ float s_y[kDcPairs][kDcCols];
    __shared__ int s_act[kDcPairs], s_off[kDcPairs];
    __shared__ uint32_t s_ids[kDcPairs];
    __shared__ int32_t s_row[kDcPairs];
    __shared__ float s_w[kDcPairs];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int P = tokens * top_k;
    const int64_t I32 = hm_pad32(I), KT = I32 / 32;
    const int64_t n0 = (int64_t)kDcCols * blockIdx.x;
    const int64_t cb = n0 >> 5;
    const int sl = (int)(n0 & 31) / kDcCols;
    // loads first, none under a branch (clamped in-range addresses; the
    // ranges are applied where the values are used): counts, then what
    // needs no routing result -- z rows, the residual, the pairs
    int cnt[NG];
    hm_load_counts<NG>(counts, experts, cnt);
    const uint32_t q4 = (uint32_t)(I32 / 4);
    float4 zv[kDcZ];
#pragma unroll
    for (int u = 0; u < kDcZ; ++u) {
        const uint32_t i = (uint32_t)tid + (uint32_t)u * kDcThreads;
        const uint32_t g = min(i / q4, (uint32_t)P - 1), k = min(4 * (i % q4), (uint32_t)I - 4);
        zv[u] = *reinterpret_cast<const float4*>(z + (int64_t)g * I + k);
    }
    const int ct = tid / kDcCols, cc = tid % kDcCols;  // combine: token ct, column n0 + cc
    const bool comb = ct < tokens && n0 + cc < H;
    float res = 0.0f;
    if (residual) res = residual[(int64_t)min(ct, tokens - 1) * H + min(n0 + cc, H - 1)];
    const int pt = min(tid, P - 1);
    const uint32_t pid = ids[pt];
    const int32_t prow = slots[pt];
    const float psc = scores[pt];
    // the active experts (ascending id), every wave: lane j < nact holds the
    // j-th, its row count and its group's first row (an exclusive prefix
    // sum, i.e. offsets[e])
    unsigned long long m[NG];
    int nact = 0;
#pragma unroll
    for (int b = 0; b < NG; ++b) {
        if ((int64_t)b * 64 + lane >= experts) cnt[b] = 0;
        m[b] = __ballot(cnt[b] > 0);
        nact += __popcll(m[b]);
    }
    nact = min(nact, kDcPairs);
    int my_act = 0, my_rows = 0;
    {
        int seen = 0;
#pragma unroll
        for (int b = 0; b < NG; ++b) {
            const int c = __popcll(m[b]);
            const int k = lane - seen;  // this lane's rank within the group
            unsigned long long mm = m[b];
            for (int i = 0; i < k && i < c; ++i) mm &= mm - 1;
            const int pos = mm ? __ffsll((long long)mm) - 1 : 0;
            const int rb = __shfl(cnt[b], pos, 64);
            if (k >= 0 && k < c) {
                my_act = b * 64 + pos;
                my_rows = rb;
            }
            seen += c;
        }
    }
    if (lane >= nact) my_rows = 0;
    int incl = my_rows;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int t = __shfl_up(incl, d, 64);
        if (lane >= d) incl += t;
    }
    const int my_off = incl - my_rows;
    // this wave's units: (expert slot, K range) -- two whole experts, or one
    // K range of 8 / nact
    const int wpe = nact >= kDcWaves ? 1 : kDcWaves / max(nact, 1);
    const int q = wave % wpe;
    const int kb0 = (int)(q * KT / wpe), nkb = (int)((q + 1) * KT / wpe) - kb0;
    const int unit_slot[2] = {nact >= kDcWaves ? wave : wave / wpe, wave + kDcWaves};
    const bool unit_on[2] = {unit_slot[0] < nact, nact >= kDcWaves && unit_slot[1] < nact};
    int unit_e[2], unit_g0[2], unit_rows[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const int sl_ = min(unit_slot[s], 63);
        unit_e[s] = __builtin_amdgcn_readfirstlane(__shfl(my_act, sl_, 64));
        unit_g0[s] = __builtin_amdgcn_readfirstlane(__shfl(my_off, sl_, 64));
        unit_rows[s] = min(__builtin_amdgcn_readfirstlane(__shfl(my_rows, sl_, 64)), kDcPairs);
    }
    // z to LDS (zero past I); the pairs' ids; the active list -- before the
    // weights are issued, so that no wait for these loads (which complete
    // in issue order) also waits for weights
#pragma unroll
    for (int u = 0; u < kDcZ; ++u) {
        const uint32_t i = (uint32_t)tid + (uint32_t)u * kDcThreads;
        if (i < (uint32_t)P * q4) *reinterpret_cast<float4*>(&s_z[4 * i]) = hm_keep_if(zv[u], 4 * (i % q4) < I);
    }
    if (tid < P) s_ids[tid] = pid;
    if (wave == 0 && lane < nact) {
        s_act[lane] = my_act;
        s_off[lane] = my_off;
    }
    __builtin_amdgcn_sched_barrier(0);  // (keeps the stores above the weight loads)
    // the weights: four K tiles per load, no branch for the first unit
    // (tiles past the K range re-read its last one, an idle wave reads
    // expert 0's; both are skipped below)
    const int tq = lane >> 4, kh = (lane >> 3) & 1, col = lane & 7;
    v4i w[2][kDcLoads];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        if (s == 1 && !unit_on[1]) continue;
        const int8_t* src = packed + hm_proj_offset(unit_e[s], 2, H, I) + cb * KT * 1024 +
                            512 * kh + 128 * sl + 16 * col;
#pragma unroll
        for (int j = 0; j < kDcLoads; ++j)
            w[s][j] = *reinterpret_cast<const v4i*>(src + (int64_t)(kb0 + min(4 * j + tq, max(nkb - 1, 0))) * 1024);
    }
    __syncthreads();
    if (tid < P) {  // hm_combine's order: the token's pairs by ascending id
        const int t = tid / top_k;
        int rank = 0;
        for (int r = 0; r < top_k; ++r) rank += s_ids[t * top_k + r] < pid;
        s_row[t * top_k + rank] = prow & (kDcPairs - 1);
        s_w[t * top_k + rank] = psc;
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        if (!unit_on[s]) continue;
        const int g0 = unit_g0[s], rows = unit_rows[s];
        for (int r = 0; r < rows; ++r) {
            float acc = 0.0f, xs = 0.0f;
            const float* zr = &s_z[(int64_t)(g0 + r) * I32 + 32 * (kb0 + tq) + 16 * kh];
            // the z values of load j + 1 are read while load j's are chained
            // (reads past the lane's K range repeat its last load's, unused)
            const int jl = max((nkb - 1 - tq) >> 2, 0);
            float4 zc[4], zn[4];
            auto read_z = [&](int j, float4 (&d)[4]) __attribute__((always_inline)) {
                const float4* xv = reinterpret_cast<const float4*>(zr + 128 * min(j, jl));
#pragma unroll
                for (int i = 0; i < 4; ++i) d[i] = xv[i];
            };
            read_z(0, zc);
#pragma unroll
            for (int j = 0; j < kDcLoads; ++j) {
                if (j + 1 < kDcLoads) read_z(j + 1, zn);
                if (4 * j + tq < nkb) {
                    float f[16];
                    tile_to_float(w[s][j], f);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float4 v = zc[i];
                        acc = __builtin_fmaf(v.x, f[4 * i], acc);
                        acc = __builtin_fmaf(v.y, f[4 * i + 1], acc);
                        acc = __builtin_fmaf(v.z, f[4 * i + 2], acc);
                        acc = __builtin_fmaf(v.w, f[4 * i + 3], acc);
                        xs += (v.x + v.y) + (v.z + v.w);
                    }
                }
                if (j + 1 < kDcLoads) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) zc[i] = zn[i];
                }
            }
            // the eight lanes of each column: K halves, then the four tiles
            acc += __shfl_xor(acc, 8, 64);
            xs += __shfl_xor(xs, 8, 64);
            acc += __shfl_xor(acc, 16, 64);
            xs += __shfl_xor(xs, 16, 64);
            acc += __shfl_xor(acc, 32, 64);
            xs += __shfl_xor(xs, 32, 64);
            if (lane < kDcCols) s_part[wave][s][r][lane] = acc;
            if (lane == 0) s_zs[wave][s][r] = xs;
        }
    }
    __syncthreads();
    // y of every grouped row for these columns: its expert's units in K order
    if (tid < P * kDcCols) {
        const int g = tid / kDcCols, c = tid % kDcCols;
        float y = 0.0f;  // no routed rows: never after a successful routing
        if (nact > 0) {
            int a = 0;
            for (int j = 1; j < nact; ++j)
                if (s_off[j] <= g) a = j;
            const int e = s_act[a], r = (g - s_off[a]) & (kDcPairs - 1);
            const int w0 = nact >= kDcWaves ? a % kDcWaves : a * wpe;
            const int su = nact >= kDcWaves ? a / kDcWaves : 0;
            float acc = 0.0f, zs = 0.0f;
            for (int j = 0; j < wpe; ++j) {
                acc += s_part[w0 + j][su][r][c];
                zs += s_zs[w0 + j][su][r];
            }
            y = __fmul_rn(__fsub_rn(acc, __fmul_rn((float)(128 + zp[e * 3 + 2]), zs)), scale[e * 3 + 2]);
        }
        s_y[g][c] = y;
        if (y_out && n0 + c < H) y_out[(int64_t)g * H + n0 + c] = y;
    }
    __syncthreads();
    // the combine of hm_combine (MoERuntime.cpp:308-325) for these columns
    if (comb) {
        float acc = 0.0f;
        for (int r = 0; r < top_k; ++r)
            acc = __fadd_rn(acc, __fmul_rn(s_w[ct * top_k + r], s_y[s_row[ct * top_k + r]][cc]));
        if (residual) acc = __fadd_rn(res, acc);
        out[(int64_t)ct * H + n0 + cc] = acc;
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
                          const int32_t* offsets, const int32_t* perm_tokens, int64_t tokens,
                          int64_t pairs, float* z, hipStream_t s) {
    if (L->experts > 1024) return HM_ERR_UNSUPPORTED;
    const int64_t slots = pairs < L->experts ? pairs : L->experts;
    const int64_t K = L->hidden, N = L->intermediate, KT = hm_pad32(K) / 32;
    if (tokens <= 2 && tokens * hm_pad32(K) <= kGvAllFloats && KT <= 32 * kGsQ) {
        // one or two tokens: every row in LDS, 8-column slices (C3-1 29.0
        // against 31.1 us per step for gemv_kernel; from four tokens on the
        // slices re-stage too many rows: C3-4 68.6 against 64.1 us)
        const dim3 grid((unsigned)((N + 7) / 8), (unsigned)slots);
        const size_t lds = (size_t)tokens * hm_pad32(K) * sizeof(float);
        const int lj = (int)((KT + kGsQ - 1) / kGsQ + 3) / 4;  // loads per wave
#define HM_GS(NG, LJ)                                                                          \
    HM_STAGE_LAUNCH(true, true, (gateup_slice_kernel<NG, LJ>), grid, dim3(kGvThreads), lds, s,   \
                    hidden, perm_tokens, K, N, L->experts,                                      \
                    static_cast<const int8_t*>(L->packed), L->scale, L->zero_point, counts,     \
                    (int)tokens, z)
#define HM_GS2(NG)                                                                             \
    do {                                                                                       \
        if (lj <= 1) HM_GS(NG, 1);                                                             \
        else if (lj <= 2) HM_GS(NG, 2);                                                        \
        else if (lj <= 4) HM_GS(NG, 4);                                                        \
        else HM_GS(NG, 8);                                                                     \
    } while (0)
        if (L->experts <= 128) HM_GS2(2);
        else if (L->experts <= 256) HM_GS2(4);
        else HM_GS2(16);
#undef HM_GS2
#undef HM_GS
        HM_LAUNCHED();
        return HM_OK;
    }
    return launch_gemv<true, 1>(hidden, perm_tokens, K, N, L, counts, offsets, slots, z, s);
}

// The decode down projection fused with the combine (P = T * k <= 16 pairs,
// I <= 768): y_out (optional) receives the expert outputs, out the block's.
bool hm_gemv_combine_ok(int64_t tokens, int32_t top_k, int64_t H, int64_t I) {
    return tokens * top_k <= kDcPairs && hm_pad32(I) / 32 <= kDcMaxTiles && I % 16 == 0 &&
           H % kDcCols == 0;
}

int hm_launch_down_combine_gemv(const hm_layer* L, const float* z, const int32_t* counts,
                                const uint32_t* ids, const int32_t* slots, const float* scores,
                                const float* residual, int64_t tokens, int32_t top_k,
                                float* y_out, float* out, hipStream_t s) {
    if (!hm_gemv_combine_ok(tokens, top_k, L->hidden, L->intermediate) || L->experts > 1024)
        return HM_ERR_UNSUPPORTED;
    const size_t lds = (size_t)tokens * top_k * hm_pad32(L->intermediate) * sizeof(float);
#define HM_DC(NG)                                                                            \
    hipLaunchKernelGGL(gemv_down_combine_kernel<NG>, dim3((unsigned)(L->hidden / kDcCols)),  \
                       dim3(kDcThreads), lds, s, z, L->intermediate, L->hidden, L->experts,  \
                       static_cast<const int8_t*>(L->packed), L->scale, L->zero_point,       \
                       counts, ids, slots, scores, residual, (int)tokens, top_k, y_out, out)
    if (L->experts <= 128) HM_DC(2);
    else if (L->experts <= 256) HM_DC(4);
    else HM_DC(16);
#undef HM_DC
    HM_LAUNCHED();
    return HM_OK;
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

// FP32 experts at decode: the shapes gemv_f32_kernel takes (K a multiple
// of 256 up to 2048 for both projections, 16-byte aligned operands).
bool hm_gemv_f32_ok(const hm_layer* L, const void* x) {
    const int64_t H = L->hidden, I = L->intermediate;
    return L->dtype == HM_DTYPE_FP32 && L->experts <= 1024 && H % 256 == 0 && I % 256 == 0 &&
           H <= 256 * kF32Mj && I <= 256 * kF32Mj && ((uintptr_t)L->packed & 15) == 0 &&
           ((uintptr_t)x & 15) == 0;
}

int hm_launch_gateup_gemv_f32(const hm_layer* L, const float* hidden, const int32_t* counts,
                              const int32_t* offsets, const int32_t* perm_tokens,
                              int64_t pairs, float* z, hipStream_t s) {
    if (!hm_gemv_f32_ok(L, hidden)) return HM_ERR_UNSUPPORTED;
    const int64_t slots = pairs < L->experts ? pairs : L->experts;
    const size_t lds = (size_t)kGvRows * L->hidden * sizeof(float);
    // K <= 1024: four columns per wave (the same registers as two at 2048)
#define HM_GF(CW, MJ)                                                                          \
    HM_STAGE_LAUNCH(true, true, (gemv_f32_kernel<true, CW, MJ>),                               \
                    dim3((unsigned)((L->intermediate + kGvWaves / 2 * CW - 1) / (kGvWaves / 2 * CW)), \
                         (unsigned)slots),                                                     \
                    dim3(kGvThreads), lds, s, hidden, perm_tokens, L->hidden, L->intermediate, \
                    L->experts, static_cast<const float*>(L->packed), L->hidden,               \
                    L->intermediate, counts, offsets, z)
    if (L->hidden <= 1024) HM_GF(4, 4);
    else HM_GF(2, 8);
#undef HM_GF
    HM_LAUNCHED();
    return HM_OK;
}

int hm_launch_down_gemv_f32(const hm_layer* L, const float* z, const int32_t* counts,
                            const int32_t* offsets, int64_t pairs, float* y, hipStream_t s) {
    if (!hm_gemv_f32_ok(L, z)) return HM_ERR_UNSUPPORTED;
    const int64_t slots = pairs < L->experts ? pairs : L->experts;
    const size_t lds = (size_t)kGvRows * L->intermediate * sizeof(float);
#define HM_GF(CW, MJ)                                                                          \
    hipLaunchKernelGGL((gemv_f32_kernel<false, CW, MJ>),                                       \
                       dim3((unsigned)((L->hidden + kGvWaves * CW - 1) / (kGvWaves * CW)),     \
                            (unsigned)slots),                                                  \
                       dim3(kGvThreads), lds, s, z, nullptr, L->intermediate, L->hidden,       \
                       L->experts, static_cast<const float*>(L->packed), L->hidden,            \
                       L->intermediate, counts, offsets, y)
    if (L->intermediate <= 1024) HM_GF(4, 4);
    else HM_GF(2, 8);
#undef HM_GF
    HM_LAUNCHED();
    return HM_OK;
}
