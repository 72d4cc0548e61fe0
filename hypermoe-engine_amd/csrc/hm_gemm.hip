// hm_gemm.hip -- expert GEMM kernels for gfx950.
//
// INT8 experts (W8A32 in the reference, CpuTensorBackend.cpp:173-186) run on
// INT8 MFMA through the integer-limb format (hm_device.h): activations are
// fixed point split into L balanced signed INT8 digit planes, one
// v_mfma_i32_32x32x32_i8 per plane, exact int32 partials, recombined in the
// epilogue (hm_gemm_mfma.hip).  The generic kernels compute the identical integers with scalar
// loops; they serve shapes the MFMA tiles do not cover and pin the MFMA
// kernels in tests (bit-for-bit).
//
// Packed expert layouts (hm_pack_layer):
//   INT8: the tile layout of hm_device.h (hm_tile_offset): per projection
//         32 x 32 tiles, each the kilobyte one MFMA B-operand load reads.
//   FP32: expert e at e*3*H*I elements, gate^T [I x H] | up^T [I x H] |
//         down^T [H x I] (K contiguous per row).
#include "hm_device.h"

#include <limits.h>

namespace {

constexpr int kBlock = 256;

// ---------------------------------------------------------------------------
// Activation rows -> digit planes (one wave per row segment).
// digits in layout lay (hm_dlay: the op-level [L][rows][n] or the block's
// X rows), scales [rows], dsum [L][rows].
// ---------------------------------------------------------------------------
template <int L>
__global__ __launch_bounds__(kBlock) void limb_quantize_rows_kernel(
    const float* __restrict__ x, int64_t rows, int64_t n,
    int8_t* __restrict__ digits, hm_dlay lay, float* __restrict__ scales,
    int32_t* __restrict__ dsum) {
    const int lane = threadIdx.x & (HM_WAVE - 1);
    const int64_t r = (int64_t)blockIdx.x * (kBlock / HM_WAVE) + threadIdx.x / HM_WAVE;
    if (r >= rows) return;
    const float* xr = x + r * n;
    float amax = 0.0f;
    for (int64_t k = lane; k < n; k += HM_WAVE) amax = fmaxf(amax, fabsf(xr[k]));
    amax = hm_wave_max_f32(amax);
    const float range = (float)hm_limb_range(L);
    const float inv = amax > 0.0f ? __fdiv_rn(range, amax) : 0.0f;
    int dl[L];
#pragma unroll
    for (int l = 0; l < L; ++l) dl[l] = 0;
    for (int64_t k = lane; k < n; k += HM_WAVE) {
        const int v = hm_fixed_point(xr[k], inv, range);
#pragma unroll
        for (int l = 0; l < L; ++l) {
            const int d = hm_digit(v, l);
            digits[hm_dlay_off(lay, l, r, k)] = (int8_t)d;
            dl[l] += d;
        }
    }
#pragma unroll
    for (int l = 0; l < L; ++l) {
        const int s = hm_wave_sum_i32(dl[l]);
        if (lane == 0 && dsum) dsum[(int64_t)l * rows + r] = s;
    }
    if (lane == 0) scales[r] = amax > 0.0f ? __fdiv_rn(amax, range) : 0.0f;
}

// The same for rows of n = 256 * nv floats (nv <= 16, 16-byte aligned):
// the row is read once into registers (lane: floats 4*(lane + 64 i) .. +3),
// reduced with DPP, and each lane stores its four digits of a plane as one
// 32-bit word.
constexpr int kQMaxV = kHmQuantMaxV;

template <int L>
__global__ __launch_bounds__(kBlock) void limb_quantize_rows_vec_kernel(
    const float* __restrict__ x, int64_t rows, int64_t n, int nv,
    int8_t* __restrict__ digits, hm_dlay lay, float* __restrict__ scales,
    int32_t* __restrict__ dsum) {
    const int lane = threadIdx.x & (HM_WAVE - 1);
    const int64_t r = (int64_t)blockIdx.x * (kBlock / HM_WAVE) + threadIdx.x / HM_WAVE;
    if (r >= rows) return;
    hm_quantize_row_wave<L>(x + r * n, nv, digits + r * lay.row, lay, scales + r,
                            dsum ? dsum + r : nullptr, rows);
}

// ---------------------------------------------------------------------------
// SwiGLU then the Z rows' digit planes: row r of gu [rows x 2n] holds the
// gate values g (columns 0..n-1) and the up values u (n..2n-1) of one grouped
// row; z = silu(g) * u (Activation.cpp:44, then the multiply) is quantised
// like any activation row (one scale per row).  One wave per row.  Digits
// in the Z layout (hm_dlay_z(L, rows)).
// ---------------------------------------------------------------------------
// rows of n = 256 * NV, 16-byte aligned: the row in registers (NV a
// template argument, so a wave holds only its own row's values)
template <int L, int NV>
__global__ __launch_bounds__(kBlock) void limb_swiglu_quantize_vec_kernel(
    const float* __restrict__ gu, int64_t rows, int64_t n,
    int8_t* __restrict__ digits, float* __restrict__ scales, int32_t* __restrict__ dsum) {
    __shared__ unsigned long long s_exp2[32];
    hm_load_exp2_table(s_exp2);
    __syncthreads();
    const int lane = threadIdx.x & (HM_WAVE - 1);
    const int64_t r = (int64_t)blockIdx.x * (kBlock / HM_WAVE) + threadIdx.x / HM_WAVE;
    if (r >= rows) return;
    const float4* g4 = reinterpret_cast<const float4*>(gu + r * 2 * n);
    const float4* u4 = reinterpret_cast<const float4*>(gu + r * 2 * n + n);
    float4 g[NV], u[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        g[i] = g4[lane + HM_WAVE * i];
        u[i] = u4[lane + HM_WAVE * i];
    }
    bool small = true;
#pragma unroll
    for (int i = 0; i < NV; ++i)
        small = small && fabsf(g[i].x) < 88.0f && fabsf(g[i].y) < 88.0f &&
                fabsf(g[i].z) < 88.0f && fabsf(g[i].w) < 88.0f;
    float4 z[NV];
    // the common path of expf holds for |g| < 88 (hm_expf_small_t); a wave
    // with any larger gate value takes the full one
    if (__all(small)) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            z[i].x = __fmul_rn(hm_silu_small_t(g[i].x, s_exp2), u[i].x);
            z[i].y = __fmul_rn(hm_silu_small_t(g[i].y, s_exp2), u[i].y);
            z[i].z = __fmul_rn(hm_silu_small_t(g[i].z, s_exp2), u[i].z);
            z[i].w = __fmul_rn(hm_silu_small_t(g[i].w, s_exp2), u[i].w);
        }
    } else {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            z[i].x = __fmul_rn(hm_silu_t(g[i].x, s_exp2), u[i].x);
            z[i].y = __fmul_rn(hm_silu_t(g[i].y, s_exp2), u[i].y);
            z[i].z = __fmul_rn(hm_silu_t(g[i].z, s_exp2), u[i].z);
            z[i].w = __fmul_rn(hm_silu_t(g[i].w, s_exp2), u[i].w);
        }
    }
    const hm_dlay lay = hm_dlay_z(L, rows);
    hm_quantize_row_values<L>(z, NV, digits + r * lay.row, lay, scales + r,
                              dsum ? dsum + r : nullptr, rows);
}

// any n: z recomputed in the digit pass
template <int L>
__global__ __launch_bounds__(kBlock) void limb_swiglu_quantize_kernel(
    const float* __restrict__ gu, int64_t rows, int64_t n,
    int8_t* __restrict__ digits, float* __restrict__ scales, int32_t* __restrict__ dsum) {
    __shared__ unsigned long long s_exp2[32];
    hm_load_exp2_table(s_exp2);
    __syncthreads();
    const int lane = threadIdx.x & (HM_WAVE - 1);
    const int64_t r = (int64_t)blockIdx.x * (kBlock / HM_WAVE) + threadIdx.x / HM_WAVE;
    if (r >= rows) return;
    const float* g = gu + r * 2 * n;
    const float* u = g + n;
    float amax = 0.0f;
    for (int64_t k = lane; k < n; k += HM_WAVE)
        amax = fmaxf(amax, fabsf(__fmul_rn(hm_silu_t(g[k], s_exp2), u[k])));
    amax = hm_wave_max_f32(amax);
    const float range = (float)hm_limb_range(L);
    const float inv = amax > 0.0f ? __fdiv_rn(range, amax) : 0.0f;
    int dl[L];
#pragma unroll
    for (int l = 0; l < L; ++l) dl[l] = 0;
    for (int64_t k = lane; k < n; k += HM_WAVE) {
        const int v = hm_fixed_point(__fmul_rn(hm_silu_t(g[k], s_exp2), u[k]), inv, range);
        const hm_dlay lay = hm_dlay_z(L, rows);
#pragma unroll
        for (int l = 0; l < L; ++l) {
            const int d = hm_digit(v, l);
            digits[hm_dlay_off(lay, l, r, k)] = (int8_t)d;
            dl[l] += d;
        }
    }
#pragma unroll
    for (int l = 0; l < L; ++l) {
        const int sm = hm_wave_sum_i32(dl[l]);
        if (lane == 0 && dsum) dsum[(int64_t)l * rows + r] = sm;
    }
    if (lane == 0) scales[r] = amax > 0.0f ? __fdiv_rn(amax, range) : 0.0f;
}

// Exact limb partials against a packed [cols x inner] INT8 matrix (test hook
// and reference semantics for the MFMA kernels).
__global__ void limb_partials_kernel(const int8_t* __restrict__ digits,
                                     int64_t rows, int64_t inner, int32_t limbs,
                                     const int8_t* __restrict__ qp, int32_t zp,
                                     int64_t cols, int32_t* __restrict__ out) {
    const int64_t idx = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    const int64_t total = (int64_t)limbs * rows * cols;
    if (idx >= total) return;
    const int64_t c = idx % cols;
    const int64_t lr = idx / cols;  // l*rows + r
    const int8_t* d = digits + lr * inner;
    const int8_t* q = qp + c * inner;
    int acc = 0;
    for (int64_t k = 0; k < inner; ++k) acc += (int)d[k] * ((int)q[k] - zp);
    out[idx] = acc;
}

// ---------------------------------------------------------------------------
// Generic INT8 expert path (any shape).  Same integers and float operation
// sequence as the MFMA kernels.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int64_t group_of_row(const int32_t* __restrict__ offsets,
                                                int64_t experts, int64_t row) {
    int64_t lo = 0, hi = experts;  // find e with offsets[e] <= row < offsets[e+1]
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) / 2;
        if (offsets[mid] <= row) lo = mid; else hi = mid;
    }
    return lo;
}

template <int L>
__global__ void gateup_generic_kernel(
    const int8_t* __restrict__ xdig, const float* __restrict__ xscale,
    int64_t tokens, int64_t H, int64_t I, int64_t experts,
    const int8_t* __restrict__ packed, const float* __restrict__ scale,
    const int32_t* __restrict__ zp, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ perm_tokens, int64_t R, float* __restrict__ gu) {
    const int64_t idx = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (idx >= R * I) return;
    const int64_t row = idx / I, col = idx % I;
    const int64_t e = group_of_row(offsets, experts, row);
    const int64_t t = perm_tokens[row];
    const int8_t* qg = packed + hm_proj_offset(e, 0, H, I);
    const int8_t* qu = packed + hm_proj_offset(e, 1, H, I);
    const int64_t H32 = hm_pad32(H);
    const int zg = zp[e * 3 + 0], zu = zp[e * 3 + 1];
    const hm_dlay lay = hm_dlay_x(L, H);
    int pg[L], pu[L];
#pragma unroll
    for (int l = 0; l < L; ++l) {
        int ag = 0, au = 0;
        for (int64_t k = 0; k < H; ++k) {
            const int64_t o = hm_tile_offset(col, k, H32);
            const int d = xdig[hm_dlay_off(lay, l, t, k)];
            ag += d * ((int)qg[o] - zg);
            au += d * ((int)qu[o] - zu);
        }
        pg[l] = ag;
        pu[l] = au;
    }
    const float sx = xscale[t];
    gu[row * 2 * I + col] = __fmul_rn(hm_recombine(pg, L), __fmul_rn(sx, scale[e * 3 + 0]));
    gu[row * 2 * I + I + col] = __fmul_rn(hm_recombine(pu, L), __fmul_rn(sx, scale[e * 3 + 1]));
}

// y[g, n] = recombine(P_l) * (s_z[g] * scale_down), P_l the exact int32
// partial of Z digit plane l over the whole row (one fixed-point scale per
// Z row, hm_launch_quantize_rows).
template <int L>
__global__ void down_generic_kernel(
    const int8_t* __restrict__ zdig, const float* __restrict__ zscale, int64_t R,
    int64_t H, int64_t I, int64_t experts, const int8_t* __restrict__ packed,
    const float* __restrict__ scale, const int32_t* __restrict__ zp,
    const int32_t* __restrict__ offsets, float* __restrict__ y) {
    const int64_t idx = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (idx >= R * H) return;
    const int64_t row = idx / H, col = idx % H;
    const int64_t e = group_of_row(offsets, experts, row);
    const int8_t* qd = packed + hm_proj_offset(e, 2, H, I);
    const int64_t I32 = hm_pad32(I);
    const int zd = zp[e * 3 + 2];
    const hm_dlay lay = hm_dlay_z(L, R);
    int p[L];
#pragma unroll
    for (int l = 0; l < L; ++l) {
        int a = 0;
        for (int64_t k = 0; k < I; ++k)
            a += (int)zdig[hm_dlay_off(lay, l, row, k)] * ((int)qd[hm_tile_offset(col, k, I32)] - zd);
        p[l] = a;
    }
    y[idx] = __fmul_rn(hm_recombine(p, L), __fmul_rn(zscale[row], scale[e * 3 + 2]));
}

// ---------------------------------------------------------------------------
// FP32 expert path (configs with FP32 weights).  Tiled FMA GEMMs, 64x64
// output tiles, 4x4 outputs per thread, K staged through LDS in steps of 16.
// ---------------------------------------------------------------------------
constexpr int kF32Tile = 64;
constexpr int kF32K = 16;

__global__ __launch_bounds__(kBlock) void gateup_f32_kernel(
    const float* __restrict__ x, int64_t H, int64_t I, int64_t experts,
    const float* __restrict__ packed, const int32_t* __restrict__ counts,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ perm_tokens,
    float* __restrict__ zf) {
    __shared__ float as[kF32K][kF32Tile + 1];
    __shared__ float bg[kF32K][kF32Tile + 1];
    __shared__ float bu[kF32K][kF32Tile + 1];
    __shared__ int32_t row_token[kF32Tile];
    const int tid = threadIdx.x;
    int64_t e, mt;
    if (!hm_locate_tile(counts, experts, kF32Tile, blockIdx.x, &e, &mt)) return;
    const int64_t g0 = offsets[e] + mt * kF32Tile;
    const int nrows = (int)min((int64_t)kF32Tile, (int64_t)counts[e] - mt * kF32Tile);
    const int64_t n0 = (int64_t)blockIdx.y * kF32Tile;
    if (tid < kF32Tile) row_token[tid] = tid < nrows ? perm_tokens[g0 + tid] : -1;
    __syncthreads();
    const float* gbase = packed + e * 3 * H * I;
    const float* ubase = gbase + H * I;
    const int tr = tid / 16, tc = tid % 16;
    float ag[4][4] = {}, au[4][4] = {};
    for (int64_t k0 = 0; k0 < H; k0 += kF32K) {
        for (int i = tid; i < kF32Tile * kF32K; i += kBlock) {
            const int r = i / kF32K, kk = i % kF32K;
            const int tok = row_token[r];
            const int64_t k = k0 + kk;
            as[kk][r] = (tok >= 0 && k < H) ? x[(int64_t)tok * H + k] : 0.0f;
            const int64_t n = n0 + r;
            const bool ok = n < I && k < H;
            bg[kk][r] = ok ? gbase[n * H + k] : 0.0f;
            bu[kk][r] = ok ? ubase[n * H + k] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kF32K; ++kk) {
            float a[4], g[4], u[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = as[kk][tr + 16 * i];
#pragma unroll
            for (int j = 0; j < 4; ++j) { g[j] = bg[kk][tc + 16 * j]; u[j] = bu[kk][tc + 16 * j]; }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    ag[i][j] = __builtin_fmaf(a[i], g[j], ag[i][j]);
                    au[i][j] = __builtin_fmaf(a[i], u[j], au[i][j]);
                }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = tr + 16 * i;
        if (r >= nrows) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t n = n0 + tc + 16 * j;
            if (n < I) zf[(g0 + r) * I + n] = __fmul_rn(hm_silu(ag[i][j]), au[i][j]);
        }
    }
}

__global__ __launch_bounds__(kBlock) void down_f32_kernel(
    const float* __restrict__ zf, int64_t H, int64_t I, int64_t experts,
    const float* __restrict__ packed, const int32_t* __restrict__ counts,
    const int32_t* __restrict__ offsets, float* __restrict__ y) {
    __shared__ float as[kF32K][kF32Tile + 1];
    __shared__ float bs[kF32K][kF32Tile + 1];
    const int tid = threadIdx.x;
    int64_t e, mt;
    if (!hm_locate_tile(counts, experts, kF32Tile, blockIdx.x, &e, &mt)) return;
    const int64_t g0 = offsets[e] + mt * kF32Tile;
    const int nrows = (int)min((int64_t)kF32Tile, (int64_t)counts[e] - mt * kF32Tile);
    const int64_t n0 = (int64_t)blockIdx.y * kF32Tile;
    const float* dbase = packed + e * 3 * H * I + 2 * H * I;
    const int tr = tid / 16, tc = tid % 16;
    float acc[4][4] = {};
    for (int64_t k0 = 0; k0 < I; k0 += kF32K) {
        for (int i = tid; i < kF32Tile * kF32K; i += kBlock) {
            const int r = i / kF32K, kk = i % kF32K;
            const int64_t k = k0 + kk;
            as[kk][r] = (r < nrows && k < I) ? zf[(g0 + r) * I + k] : 0.0f;
            const int64_t n = n0 + r;
            bs[kk][r] = (n < H && k < I) ? dbase[n * I + k] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kF32K; ++kk) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = as[kk][tr + 16 * i];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = bs[kk][tc + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = tr + 16 * i;
        if (r >= nrows) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t n = n0 + tc + 16 * j;
            if (n < H) y[(g0 + r) * H + n] = acc[i][j];
        }
    }
}

// ---------------------------------------------------------------------------
// Op-level GEMMs on the reference's [K x N] weight layout.
// ---------------------------------------------------------------------------
// Reference mode: one lane per output, K ascending, float multiply then add
// with the dequantised weight float(q - zp) * scale: the reference loop
// (CpuTensorBackend.cpp:173-186) operation for operation, hence bit-exact.
__global__ void w8a32_reference_kernel(const float* __restrict__ x,
                                       const int8_t* __restrict__ q, float scale,
                                       int32_t zp, float* __restrict__ y,
                                       int64_t rows, int64_t inner, int64_t cols) {
    const int64_t idx = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (idx >= rows * cols) return;
    const int64_t r = idx / cols, c = idx % cols;
    float sum = 0.0f;
    for (int64_t k = 0; k < inner; ++k) {
        const float w = __fmul_rn((float)((int)q[k * cols + c] - zp), scale);
        sum = __fadd_rn(sum, __fmul_rn(x[r * inner + k], w));
    }
    y[idx] = sum;
}

// Cooperative mode: bounded split-K.  Grid (ceil(N/64), M, P); partition p
// covers the balanced K range [p*base + min(p, rem), ...); lane = column;
// wave w accumulates k = begin + w, begin + w + 4, ... in order; the four
// wave sums are added in fixed order ((w0 + w1) + w2) + w3.  P > 1 writes
// partials that a second kernel adds in ascending p.  Deterministic.
__global__ __launch_bounds__(kBlock) void w8a32_coop_kernel(
    const float* __restrict__ x, const int8_t* __restrict__ q, float scale,
    int32_t zp, float* __restrict__ out, int64_t rows, int64_t inner,
    int64_t cols, int64_t parts) {
    __shared__ float red[4][HM_WAVE];
    const int lane = threadIdx.x & (HM_WAVE - 1);
    const int wave = threadIdx.x / HM_WAVE;
    const int64_t c = (int64_t)blockIdx.x * HM_WAVE + lane;
    const int64_t r = blockIdx.y;
    const int64_t p = blockIdx.z;
    const int64_t base = inner / parts, rem = inner % parts;
    const int64_t begin = p * base + (p < rem ? p : rem);
    const int64_t end = begin + base + (p < rem ? 1 : 0);
    float sum = 0.0f;
    if (c < cols) {
        for (int64_t k = begin + wave; k < end; k += 4) {
            const float w = __fmul_rn((float)((int)q[k * cols + c] - zp), scale);
            sum = __fadd_rn(sum, __fmul_rn(x[r * inner + k], w));
        }
    }
    red[wave][lane] = sum;
    __syncthreads();
    if (wave == 0 && c < cols) {
        const float s = __fadd_rn(__fadd_rn(__fadd_rn(red[0][lane], red[1][lane]), red[2][lane]),
                                  red[3][lane]);
        out[(p * rows + r) * cols + c] = s;
    }
}

__global__ void reduce_parts_kernel(const float* __restrict__ parts_in, int64_t parts,
                                    int64_t count, float* __restrict__ y) {
    const int64_t idx = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (idx >= count) return;
    float s = parts_in[idx];
    for (int64_t p = 1; p < parts; ++p) s = __fadd_rn(s, parts_in[p * count + idx]);
    y[idx] = s;
}

__global__ __launch_bounds__(kBlock) void matmul_f32_kernel(
    const float* __restrict__ x, const float* __restrict__ w, float* __restrict__ y,
    int64_t rows, int64_t inner, int64_t cols) {
    __shared__ float as[kF32K][kF32Tile + 1];
    __shared__ float bs[kF32K][kF32Tile + 1];
    const int tid = threadIdx.x;
    const int64_t m0 = (int64_t)blockIdx.x * kF32Tile, n0 = (int64_t)blockIdx.y * kF32Tile;
    const int tr = tid / 16, tc = tid % 16;
    float acc[4][4] = {};
    for (int64_t k0 = 0; k0 < inner; k0 += kF32K) {
        for (int i = tid; i < kF32Tile * kF32K; i += kBlock) {
            const int r = i / kF32K, kk = i % kF32K;
            const int64_t k = k0 + kk;
            as[kk][r] = (m0 + r < rows && k < inner) ? x[(m0 + r) * inner + k] : 0.0f;
            const int kk2 = i / kF32Tile, cc = i % kF32Tile;
            const int64_t k2 = k0 + kk2;
            bs[kk2][cc] = (k2 < inner && n0 + cc < cols) ? w[k2 * cols + n0 + cc] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kF32K; ++kk) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = as[kk][tr + 16 * i];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = bs[kk][tc + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t r = m0 + tr + 16 * i, c = n0 + tc + 16 * j;
            if (r < rows && c < cols) y[r * cols + c] = acc[i][j];
        }
}

// [K x N] -> [N x K] transpose of one projection (32x32 LDS tiles).
template <typename T>
__global__ void transpose_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                 int64_t K, int64_t N) {
    __shared__ T tile[32][33];
    const int64_t k0 = (int64_t)blockIdx.y * 32, n0 = (int64_t)blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    for (int i = ty; i < 32; i += 8) {
        const int64_t k = k0 + i, n = n0 + tx;
        if (k < K && n < N) tile[i][tx] = src[k * N + n];
    }
    __syncthreads();
    for (int i = ty; i < 32; i += 8) {
        const int64_t n = n0 + i, k = k0 + tx;
        if (k < K && n < N) dst[n * K + k] = tile[tx][i];
    }
}

// INT8 projection [K x N] (row-major, the reference payload) -> tiles
// (hm_tile_offset), zero-padded to N32 x K32.  One workgroup per tile: the
// 32 x 32 source block through LDS, then the kilobyte in lane order.
// blockIdx.x: tile of the projection (cb * K32/32 + kb), blockIdx.y: 3e + p.
__global__ __launch_bounds__(256) void pack_tiles_i8_kernel(const int8_t* __restrict__ src,
                                                            int8_t* __restrict__ dst, int64_t H,
                                                            int64_t I) {
    __shared__ int8_t t[32][33];
    const int64_t ep = blockIdx.y;
    const int p = (int)(ep % 3);
    const int64_t K = p < 2 ? H : I, N = p < 2 ? I : H;
    const int64_t K32 = hm_pad32(K);
    const int64_t cb = blockIdx.x / (K32 >> 5), kb = blockIdx.x % (K32 >> 5);
    const int8_t* s = src + ep * H * I;
    const int tid = threadIdx.x;
    const int kr = tid >> 3, nc = (tid & 7) * 4;
    const int64_t k = 32 * kb + kr;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t n = 32 * cb + nc + j;
        t[kr][nc + j] = (k < K && n < N) ? s[k * N + n] : (int8_t)0;
    }
    __syncthreads();
    if (tid < 64) {
        const int nl = tid & 31, k0 = 16 * (tid >> 5);
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            w[q] = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) w[q] |= (uint32_t)(uint8_t)t[k0 + 4 * q + b][nl] << (8 * b);
        }
        int8_t* d = dst + hm_proj_offset(ep / 3, p, H, I) + (int64_t)blockIdx.x * 1024 + 16 * tid;
        *reinterpret_cast<uint4*>(d) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

}  // namespace

// ===========================================================================
// Launchers used by the block entry (hm_block.hip) and the C ABI.
// ===========================================================================
// Rows -> digit planes.
static int quantize_rows(const float* x, int64_t rows, int64_t n, int32_t limbs,
                         int8_t* digits, const hm_dlay& lay, float* scales, int32_t* dsum,
                         hipStream_t stream) {
    if (rows == 0) return HM_OK;
    const dim3 grid((unsigned)((rows + 3) / 4));
    const int64_t nv = n / 256;
    if (n % 256 == 0 && nv >= 1 && nv <= kQMaxV && (uintptr_t)x % 16 == 0 && (uintptr_t)digits % 4 == 0) {
#define HM_QV(LV) HM_STAGE_LAUNCH(false, false, limb_quantize_rows_vec_kernel<LV>, grid, dim3(kBlock), 0, stream, \
                                  x, rows, n, (int)nv, digits, lay, scales, dsum)
        switch (limbs) {
        case 1: HM_QV(1); break;
        case 2: HM_QV(2); break;
        case 3: HM_QV(3); break;
        default: return HM_ERR_INVALID;
        }
#undef HM_QV
        HM_LAUNCHED();
        return HM_OK;
    }
#define HM_QS(LV) HM_STAGE_LAUNCH(false, false, limb_quantize_rows_kernel<LV>, grid, dim3(kBlock), 0, stream, \
                                  x, rows, n, digits, lay, scales, dsum)
    switch (limbs) {
    case 1: HM_QS(1); break;
    case 2: HM_QS(2); break;
    case 3: HM_QS(3); break;
    default: return HM_ERR_INVALID;
    }
#undef HM_QS
    HM_LAUNCHED();
    return HM_OK;
}

// The block's token rows in the X digit layout (hm_dlay_x).
int hm_launch_quantize_rows(const float* x, int64_t rows, int64_t n, int32_t limbs,
                            int8_t* digits, float* scales, int32_t* dsum,
                            hipStream_t stream) {
    return quantize_rows(x, rows, n, limbs, digits, hm_dlay_x(limbs, n), scales, dsum, stream);
}

// gu [rows x 2n] (g | u per row) -> z = silu(g) * u -> digit planes in the
// Z layout (hm_dlay_z); the last launch of the gate/up stage (its end closes
// an armed stage timer).
static int swiglu_quantize_rows(const float* gu, int64_t rows, int64_t n, int32_t limbs,
                                int8_t* digits, float* scales, int32_t* dsum,
                                hipStream_t stream) {
    if (rows == 0) return HM_OK;
    if (limbs < 1 || limbs > 3) return HM_ERR_INVALID;
    const dim3 grid((unsigned)((rows + 3) / 4));
    const int64_t nv = n / 256;
    const bool vec = n % 256 == 0 && (uintptr_t)gu % 16 == 0 && (uintptr_t)digits % 4 == 0;
#define HM_SQ(LV, NV) HM_STAGE_LAUNCH(false, true, (limb_swiglu_quantize_vec_kernel<LV, NV>), grid, \
                                      dim3(kBlock), 0, stream, gu, rows, n, digits, scales, dsum)
#define HM_SQL(NV)                                          \
    do {                                                    \
        if (limbs == 1) HM_SQ(1, NV);                       \
        else if (limbs == 2) HM_SQ(2, NV);                  \
        else HM_SQ(3, NV);                                  \
    } while (0)
    if (vec && nv == 1) HM_SQL(1);
    else if (vec && nv == 2) HM_SQL(2);
    else if (vec && nv == 3) HM_SQL(3);
    else if (vec && nv == 4) HM_SQL(4);
    else if (vec && nv == 6) HM_SQL(6);
    else if (vec && nv == 8) HM_SQL(8);
    else {
#define HM_SG(LV) HM_STAGE_LAUNCH(false, true, limb_swiglu_quantize_kernel<LV>, grid, dim3(kBlock), 0, \
                                  stream, gu, rows, n, digits, scales, dsum)
        if (limbs == 1) HM_SG(1);
        else if (limbs == 2) HM_SG(2);
        else HM_SG(3);
#undef HM_SG
    }
#undef HM_SQL
#undef HM_SQ
    HM_LAUNCHED();
    return HM_OK;
}

bool hm_mfma_gateup_ok(int64_t H, int64_t I, int64_t E, int32_t limbs);
bool hm_mfma_down_ok(int64_t H, int64_t I, int64_t E, int32_t limbs);
int hm_launch_gateup_i8_mfma(const hm_layer* layer, int32_t limbs, const int8_t* xdig,
                             const float* xscale, const int32_t* xdsum, int64_t tokens,
                             const int32_t* counts, const int32_t* offsets,
                             const int32_t* perm_tokens, int64_t R, float* gu, bool split_k,
                             hipStream_t stream);
int hm_launch_down_i8_mfma(const hm_layer* layer, int32_t limbs, const int32_t* counts,
                           const int32_t* offsets, int64_t R, const int8_t* zdig,
                           const float* zscale, const int32_t* zdsum, float* y, bool split_k,
                           hipStream_t stream);

int64_t hm_max_tiles(int64_t pairs, int64_t experts, int64_t tile_m) {
    return (pairs < experts ? pairs : experts) + pairs / tile_m;
}

// INT8 expert GEMMs: gate/up (the dequantised gate and up values of every
// grouped row into gu [R x 2I]), z = silu(g) * u and the Z rows' fixed-point
// digits (one scale per row, the same quantiser as the activations), then
// down.  xdig/xscale/xdsum: the token rows' digits
// (hm_launch_quantize_rows over all tokens, or the prefill router's select
// kernel).  The MFMA kernels (hm_gemm_mfma.hip) where the shape allows, the
// generic kernels otherwise; both compute the same integers and the same
// float operation sequence.
bool hm_use_mfma_gateup(const hm_layer* layer, int32_t lx, bool force_generic) {
    return !force_generic && hm_mfma_gateup_ok(layer->hidden, layer->intermediate, layer->experts, lx);
}
bool hm_use_mfma_down(const hm_layer* layer, int32_t lz, bool force_generic) {
    return !force_generic && hm_mfma_down_ok(layer->hidden, layer->intermediate, layer->experts, lz);
}

int hm_launch_gateup_i8(const hm_layer* layer, int32_t lx, int32_t lz, const int8_t* xdig,
                        const float* xscale, const int32_t* xdsum, int64_t tokens,
                        const int32_t* counts, const int32_t* offsets,
                        const int32_t* perm_tokens, int64_t R, int8_t* zdig, float* zscale,
                        int32_t* zdsum, float* gu, bool force_generic, bool split_k,
                        hipStream_t stream) {
    const int64_t H = layer->hidden, I = layer->intermediate, E = layer->experts;
    const int8_t* packed = static_cast<const int8_t*>(layer->packed);
    if (R == 0) return HM_OK;
    // the MFMA kernels, or the generic ones where the shape (or a 32-bit
    // buffer offset) rules them out
    int rc = hm_use_mfma_gateup(layer, lx, force_generic)
                 ? hm_launch_gateup_i8_mfma(layer, lx, xdig, xscale, xdsum, tokens, counts,
                                            offsets, perm_tokens, R, gu, split_k, stream)
                 : HM_ERR_UNSUPPORTED;
    if (rc == HM_ERR_UNSUPPORTED) {
        rc = HM_OK;
        const unsigned g_gu = (unsigned)((R * I + kBlock - 1) / kBlock);
#define HM_GU(LV)                                                                               \
        HM_STAGE_LAUNCH(true, false, gateup_generic_kernel<LV>, dim3(g_gu), dim3(kBlock), 0, stream, \
                        xdig, xscale, tokens, H, I, E, packed, layer->scale, layer->zero_point,   \
                        offsets, perm_tokens, R, gu)
        switch (lx) {
        case 1: HM_GU(1); break;
        case 2: HM_GU(2); break;
        case 3: HM_GU(3); break;
        default: return HM_ERR_INVALID;
        }
#undef HM_GU
        HM_LAUNCHED();
    }
    if (rc) return rc;
    // the stage's last launch (its end closes the timed span when armed)
    return swiglu_quantize_rows(gu, R, I, lz, zdig, zscale, zdsum, stream);
}

int hm_launch_down_i8(const hm_layer* layer, int32_t lx, int32_t lz, const int32_t* counts,
                      const int32_t* offsets, int64_t R, const int8_t* zdig,
                      const float* zscale, const int32_t* zdsum, float* y,
                      bool force_generic, bool split_k, hipStream_t stream) {
    const int64_t H = layer->hidden, I = layer->intermediate, E = layer->experts;
    const int8_t* packed = static_cast<const int8_t*>(layer->packed);
    if (R == 0) return HM_OK;
    if (hm_use_mfma_down(layer, lz, force_generic)) {
        const int rc = hm_launch_down_i8_mfma(layer, lz, counts, offsets, R, zdig, zscale, zdsum,
                                              y, split_k, stream);
        if (rc != HM_ERR_UNSUPPORTED) return rc;
    }
    const unsigned g_dn = (unsigned)((R * H + kBlock - 1) / kBlock);
#define HM_DN(LV)                                                                       \
    hipLaunchKernelGGL(down_generic_kernel<LV>, dim3(g_dn), dim3(kBlock), 0, stream,     \
                       zdig, zscale, R, H, I, E, packed, layer->scale, layer->zero_point,\
                       offsets, y)
    switch (lz) {
    case 1: HM_DN(1); break;
    case 2: HM_DN(2); break;
    case 3: HM_DN(3); break;
    default: return HM_ERR_INVALID;
    }
#undef HM_DN
    HM_LAUNCHED();
    return HM_OK;
}

bool hm_f32_mfma_gateup_ok(int64_t H, int64_t I);
bool hm_f32_mfma_down_ok(int64_t H, int64_t I);
int hm_launch_gateup_f32_mfma(const hm_layer* L, const float* hidden, const int32_t* counts,
                              const int32_t* offsets, const int32_t* perm_tokens, int64_t R,
                              int64_t max_tiles, float* z, hipStream_t stream);
int hm_launch_down_f32_mfma(const hm_layer* L, const float* z, const int32_t* counts,
                            const int32_t* offsets, int64_t R, int64_t max_tiles, float* y,
                            hipStream_t stream);

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// FP32 experts: the matrix-core tiles (hm_gemm_f32_mfma.hip) where the
// shape allows, else the FMA tiles above.
int hm_launch_gateup_f32(const hm_layer* layer, const float* hidden, const int32_t* counts,
                         const int32_t* offsets, const int32_t* perm_tokens, int64_t R,
                         float* zf, hipStream_t stream) {
    const int64_t H = layer->hidden, I = layer->intermediate, E = layer->experts;
    if (R == 0) return HM_OK;
    if (hm_f32_mfma_gateup_ok(H, I) && aligned16(hidden) && aligned16(layer->packed))
        return hm_launch_gateup_f32_mfma(layer, hidden, counts, offsets, perm_tokens, R,
                                         hm_max_tiles(R, E, 64), zf, stream);
    const dim3 g1((unsigned)hm_max_tiles(R, E, kF32Tile), (unsigned)((I + kF32Tile - 1) / kF32Tile));
    HM_STAGE_LAUNCH(true, true, gateup_f32_kernel, g1, dim3(kBlock), 0, stream, hidden, H, I, E,
                    static_cast<const float*>(layer->packed), counts, offsets, perm_tokens, zf);
    HM_LAUNCHED();
    return HM_OK;
}

int hm_launch_down_f32(const hm_layer* layer, const int32_t* counts, const int32_t* offsets,
                       int64_t R, const float* zf, float* y, hipStream_t stream) {
    const int64_t H = layer->hidden, I = layer->intermediate, E = layer->experts;
    if (R == 0) return HM_OK;
    if (hm_f32_mfma_down_ok(H, I) && aligned16(zf) && aligned16(layer->packed))
        return hm_launch_down_f32_mfma(layer, zf, counts, offsets, R, hm_max_tiles(R, E, 64), y,
                                       stream);
    const dim3 g2((unsigned)hm_max_tiles(R, E, kF32Tile), (unsigned)((H + kF32Tile - 1) / kF32Tile));
    hipLaunchKernelGGL(down_f32_kernel, g2, dim3(kBlock), 0, stream, zf, H, I, E,
                       static_cast<const float*>(layer->packed), counts, offsets, y);
    HM_LAUNCHED();
    return HM_OK;
}

extern "C" {

int hm_limb_quantize_rows(const float* x, int64_t rows, int64_t inner, int32_t limbs,
                          int8_t* digits, float* scales, void* stream) {
    HM_REQUIRE(x && digits && scales && rows >= 0 && inner > 0);
    HM_REQUIRE(limbs >= 1 && limbs <= 3);
    return quantize_rows(x, rows, inner, limbs, digits, hm_dlay_planes(rows, inner), scales,
                         nullptr, hm_stream(stream));
}

int hm_limb_partials(const int8_t* digits, int64_t rows, int64_t inner, int32_t limbs,
                     const int8_t* q_packed, int32_t zp, int64_t cols,
                     int32_t* partials, void* stream) {
    HM_REQUIRE(digits && q_packed && partials && rows >= 0 && inner > 0 && cols > 0);
    HM_REQUIRE(limbs >= 1 && limbs <= 3 && zp >= -128 && zp <= 127);
    if (inner > 65536) return HM_ERR_OVERFLOW;  // |partial| <= inner*128*255 < 2^31
    const int64_t total = (int64_t)limbs * rows * cols;
    if (total == 0) return HM_OK;
    hipLaunchKernelGGL(limb_partials_kernel, dim3((unsigned)((total + kBlock - 1) / kBlock)),
                       dim3(kBlock), 0, hm_stream(stream), digits, rows, inner, limbs,
                       q_packed, zp, cols, partials);
    HM_LAUNCHED();
    return HM_OK;
}

int hm_plan_int8_gemm(int64_t rows, int64_t inner, int64_t cols, int32_t mode,
                      hm_int8_gemm_plan* plan) {
    HM_REQUIRE(plan && rows > 0 && inner > 0 && cols > 0);
    HM_REQUIRE(mode >= 0 && mode <= 2);
    // Int8GemmPlan.cpp:31-36: overflow guards on M*N, M*K, K*N
    if (rows > INT64_MAX / cols || rows > INT64_MAX / inner || inner > INT64_MAX / cols)
        return HM_ERR_OVERFLOW;
    const int implementation = mode == 0 ? ((inner >= 256 && cols >= 64) ? 2 : 1) : mode;
    plan->implementation = implementation;
    if (implementation == 1) {
        plan->partitions = 1;
        plan->blocks = (rows * cols + kBlock - 1) / kBlock;
        plan->scratch_elements = 0;
    } else {
        const int64_t p = (inner + 511) / 512;
        plan->partitions = p < 8 ? p : 8;
        const int64_t col_blocks = (cols + HM_WAVE - 1) / HM_WAVE;
        if (rows > INT64_MAX / plan->partitions ||
            rows * plan->partitions > INT64_MAX / col_blocks) return HM_ERR_OVERFLOW;
        plan->blocks = rows * plan->partitions * col_blocks;
        plan->scratch_elements = plan->partitions > 1 ? rows * cols * plan->partitions : 0;
    }
    if (plan->blocks > INT_MAX) return HM_ERR_OVERFLOW;
    return HM_OK;
}

int hm_matmul_w8a32(const float* x, const int8_t* q, float scale, int32_t zp,
                    float* y, int64_t rows, int64_t inner, int64_t cols, int32_t mode,
                    float* scratch, size_t scratch_bytes, void* stream) {
    // quantization::validateParameters (Quantization.cpp:24-35)
    HM_REQUIRE(std::isfinite(scale) && scale > 0.0f && zp >= -128 && zp <= 127);
    HM_REQUIRE(x && q && y);
    HM_REQUIRE((const void*)x != (const void*)y && (const void*)q != (const void*)y);
    hm_int8_gemm_plan plan;
    const int rc = hm_plan_int8_gemm(rows, inner, cols, mode, &plan);
    if (rc) return rc;
    hipStream_t s = hm_stream(stream);
    if (plan.implementation == 1) {
        hipLaunchKernelGGL(w8a32_reference_kernel, dim3((unsigned)plan.blocks), dim3(kBlock),
                           0, s, x, q, scale, zp, y, rows, inner, cols);
        HM_LAUNCHED();
        return HM_OK;
    }
    if (rows > 65535) return HM_ERR_UNSUPPORTED;
    const dim3 grid((unsigned)((cols + HM_WAVE - 1) / HM_WAVE), (unsigned)rows,
                    (unsigned)plan.partitions);
    if (plan.partitions == 1) {
        hipLaunchKernelGGL(w8a32_coop_kernel, grid, dim3(kBlock), 0, s, x, q, scale, zp, y,
                           rows, inner, cols, plan.partitions);
        HM_LAUNCHED();
        return HM_OK;
    }
    HM_REQUIRE(scratch && scratch_bytes >= (size_t)plan.scratch_elements * sizeof(float));
    hipLaunchKernelGGL(w8a32_coop_kernel, grid, dim3(kBlock), 0, s, x, q, scale, zp, scratch,
                       rows, inner, cols, plan.partitions);
    HM_LAUNCHED();
    const int64_t count = rows * cols;
    hipLaunchKernelGGL(reduce_parts_kernel, dim3((unsigned)((count + kBlock - 1) / kBlock)),
                       dim3(kBlock), 0, s, scratch, plan.partitions, count, y);
    HM_LAUNCHED();
    return HM_OK;
}

int hm_matmul_f32(const float* x, const float* w, float* y, int64_t rows, int64_t inner,
                  int64_t cols, void* stream) {
    HM_REQUIRE(x && w && y && rows > 0 && inner > 0 && cols > 0);
    HM_REQUIRE((const void*)x != (const void*)y && (const void*)w != (const void*)y);
    const dim3 grid((unsigned)((rows + kF32Tile - 1) / kF32Tile),
                    (unsigned)((cols + kF32Tile - 1) / kF32Tile));
    hipLaunchKernelGGL(matmul_f32_kernel, grid, dim3(kBlock), 0, hm_stream(stream), x, w, y,
                       rows, inner, cols);
    HM_LAUNCHED();
    return HM_OK;
}

size_t hm_packed_layer_bytes(int64_t experts, int64_t hidden, int64_t intermediate,
                             int32_t dtype) {
    if (experts <= 0 || hidden <= 0 || intermediate <= 0) return 0;
    if (dtype == HM_DTYPE_INT8) return (size_t)experts * 3 * (size_t)hm_proj_bytes(hidden, intermediate);
    if (dtype == HM_DTYPE_FP32) return (size_t)experts * 3 * (size_t)hidden * (size_t)intermediate * 4;
    return 0;
}

int hm_pack_layer(const void* src, int64_t experts, int64_t hidden, int64_t intermediate,
                  int32_t dtype, void* dst, void* stream) {
    HM_REQUIRE(src && dst && src != dst && experts > 0 && hidden > 0 && intermediate > 0);
    HM_REQUIRE(dtype == HM_DTYPE_INT8 || dtype == HM_DTYPE_FP32);
    const int64_t H = hidden, I = intermediate;
    hipStream_t s = hm_stream(stream);
    if (dtype == HM_DTYPE_INT8) {
        const int64_t tiles = hm_proj_bytes(H, I) / 1024;
        if (tiles > INT_MAX || 3 * experts > 65535) return HM_ERR_UNSUPPORTED;
        hipLaunchKernelGGL(pack_tiles_i8_kernel, dim3((unsigned)tiles, (unsigned)(3 * experts)),
                           dim3(256), 0, s, static_cast<const int8_t*>(src),
                           static_cast<int8_t*>(dst), H, I);
        HM_LAUNCHED();
        return HM_OK;
    }
    for (int64_t e = 0; e < experts; ++e) {
        for (int p = 0; p < 3; ++p) {
            const int64_t K = p < 2 ? H : I, N = p < 2 ? I : H;
            const int64_t off = e * 3 * H * I + p * H * I;
            const dim3 grid((unsigned)((N + 31) / 32), (unsigned)((K + 31) / 32));
            hipLaunchKernelGGL(transpose_kernel<float>, grid, dim3(kBlock), 0, s,
                               static_cast<const float*>(src) + off,
                               static_cast<float*>(dst) + off, K, N);
            HM_LAUNCHED();
        }
    }
    return HM_OK;
}

}  // extern "C"
