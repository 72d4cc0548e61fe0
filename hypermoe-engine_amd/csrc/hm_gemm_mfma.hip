// hm_gemm_mfma.hip -- grouped INT8-MFMA expert GEMMs for gfx950.
//
// Both kernels run 512-thread workgroups (8 wave64s) over one tile of one
// expert's grouped rows.  The activation operand is L fixed-point digit
// planes (hm_device.h); every digit plane meets the same weight fragment in
// one v_mfma_i32_16x16x64_i8, so the int32 partial of each plane is exact.
//
// Data movement per 64-wide K step: every thread issues its global loads for
// step s+1 into registers, the waves run the MFMAs of step s out of one LDS
// buffer, the prefetched registers go to the other buffer, one barrier.
// LDS rows are padded to 80 bytes: the 16 lanes that read one 16-byte column
// of 16 consecutive rows then hit 16 disjoint groups of 4 banks.
//
// MFMA operand layout (v_mfma_i32_16x16x64_i8): lane l supplies 16 bytes of
// row (l % 16) of A and of column (l % 16) of B, holding K elements
// 16*(l/16) .. 16*(l/16)+15 of the step in both operands; the 4 int32 results
// of lane l are rows 4*(l/16) + 0..3 of column l % 16.
#include "hm_device.h"

#include <limits.h>

namespace {

constexpr int kThreads = 512;
constexpr int kStepK = 64;
constexpr int kRow = kStepK + 16;   // padded LDS row, bytes
constexpr int kZBlock = 128;
constexpr int kGateUpN = 128;       // columns per projection per gate/up tile
constexpr int kDownN = 256;         // output columns per down tile

typedef int v4i __attribute__((ext_vector_type(4)));

template <int L>
struct Tiles {
    // rows per workgroup: 2 row groups of waves x WM 16-row subtiles
    static constexpr int WM = L >= 3 ? 2 : 4;
    static constexpr int BM = 2 * 16 * WM;
};

__device__ __forceinline__ v4i ld16(const int8_t* p) {
    return *reinterpret_cast<const v4i*>(p);
}
__device__ __forceinline__ void st16(int8_t* p, v4i v) { *reinterpret_cast<v4i*>(p) = v; }

// ---------------------------------------------------------------------------
// gate/up: tile = BM grouped rows x (128 gate + 128 up) columns.
// wave (wm, wn) = (wave / 4, wave % 4): rows [wm*BM/2, +BM/2), gate and up
// columns [32 wn, 32 wn + 32) of the tile.  Epilogue: z = silu(g) * u, the
// 128-column fixed-point segment of each Z row is quantised to L digits.
// ---------------------------------------------------------------------------
template <int L>
__global__ __launch_bounds__(kThreads) void gateup_mfma_kernel(
    const int8_t* __restrict__ xdig, const float* __restrict__ xscale,
    const int32_t* __restrict__ xdsum, int64_t tokens, int64_t H, int64_t I,
    int64_t experts, const int8_t* __restrict__ packed,
    const float* __restrict__ scale, const int32_t* __restrict__ zp,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ perm_tokens, int64_t R, int8_t* __restrict__ zdig,
    float* __restrict__ zscale, int32_t* __restrict__ zdsum) {
    constexpr int WM = Tiles<L>::WM, BM = Tiles<L>::BM;
    constexpr int A_CHUNKS = L * BM * 4;   // 16-byte chunks of A per step
    constexpr int B_CHUNKS = 256 * 4;      // 256 weight rows x 4 chunks
    __shared__ __attribute__((aligned(16))) int8_t lds_a[2][L][BM][kRow];
    __shared__ __attribute__((aligned(16))) int8_t lds_b[2][256][kRow];
    __shared__ int32_t row_token[BM];
    __shared__ float red[BM][4];
    __shared__ int red_i[L][BM][4];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 2, wn = wave & 3;
    int64_t e, mt;
    if (!hm_locate_tile(counts, experts, BM, blockIdx.x, &e, &mt)) return;
    const int64_t g0 = offsets[e] + mt * BM;
    const int nrows = (int)min((int64_t)BM, (int64_t)counts[e] - mt * BM);
    const int64_t n0 = (int64_t)blockIdx.y * kGateUpN;
    if (tid < BM) row_token[tid] = tid < nrows ? perm_tokens[g0 + tid] : -1;
    __syncthreads();

    // global -> register staging assignments
    const int8_t* ebase = packed + e * 3 * H * I;
    const int8_t* a_src[(A_CHUNKS + kThreads - 1) / kThreads];
    int a_dst[(A_CHUNKS + kThreads - 1) / kThreads];
#pragma unroll
    for (int c = 0; c < (A_CHUNKS + kThreads - 1) / kThreads; ++c) {
        const int chunk = tid + c * kThreads;
        a_src[c] = nullptr;
        a_dst[c] = -1;
        if (chunk < A_CHUNKS) {
            const int l = chunk / (BM * 4), rem = chunk % (BM * 4);
            const int r = rem >> 2, seg = rem & 3;
            const int tok = row_token[r];
            a_dst[c] = (l * BM + r) * kRow + 16 * seg;
            if (tok >= 0) a_src[c] = xdig + ((int64_t)l * tokens + tok) * H + 16 * seg;
        }
    }
    const int8_t* b_src[2];
    int b_dst[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int chunk = tid + c * kThreads;  // < 1024 = B_CHUNKS
        const int r = chunk >> 2, seg = chunk & 3;
        const int64_t col = n0 + (r & 127);
        b_src[c] = ebase + (r >> 7) * H * I + col * H + 16 * seg;
        b_dst[c] = r * kRow + 16 * seg;
    }
    static_assert(B_CHUNKS == 2 * kThreads, "two weight chunks per thread");

    constexpr int NA = (A_CHUNKS + kThreads - 1) / kThreads;
    v4i ra[NA], rb[2];
    auto fetch = [&](int64_t k0) {
#pragma unroll
        for (int c = 0; c < NA; ++c) ra[c] = a_src[c] ? ld16(a_src[c] + k0) : v4i{0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < 2; ++c) rb[c] = ld16(b_src[c] + k0);
    };
    auto stash = [&](int buf) {
        int8_t* a = &lds_a[buf][0][0][0];
#pragma unroll
        for (int c = 0; c < NA; ++c) if (a_dst[c] >= 0) st16(a + a_dst[c], ra[c]);
        int8_t* b = &lds_b[buf][0][0];
#pragma unroll
        for (int c = 0; c < 2; ++c) st16(b + b_dst[c], rb[c]);
    };

    v4i acc[WM][4][L];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int l = 0; l < L; ++l) acc[i][j][l] = v4i{0, 0, 0, 0};

    const int nk = (int)(H / kStepK);
    fetch(0);
    stash(0);
    __syncthreads();
    const int arow = wm * (BM / 2) + (lane & 15);
    const int kofs = 16 * (lane >> 4);
    for (int ks = 0; ks < nk; ++ks) {
        const int buf = ks & 1;
        if (ks + 1 < nk) fetch((int64_t)(ks + 1) * kStepK);
        v4i b[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int brow = (j >> 1) * 128 + 32 * wn + 16 * (j & 1) + (lane & 15);
            b[j] = ld16(&lds_b[buf][brow][kofs]);
        }
#pragma unroll
        for (int i = 0; i < WM; ++i) {
#pragma unroll
            for (int l = 0; l < L; ++l) {
                const v4i a = ld16(&lds_a[buf][l][arow + 16 * i][kofs]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[i][j][l] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[j], acc[i][j][l], 0, 0, 0);
                }
            }
        }
        if (ks + 1 < nk) stash(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue -------------------------------------------------------
    const float sg = scale[e * 3 + 0], su = scale[e * 3 + 1];
    const int zg = zp[e * 3 + 0], zu = zp[e * 3 + 1], zd = zp[e * 3 + 2];
    float z[WM][2][4];
#pragma unroll
    for (int i = 0; i < WM; ++i) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int r = wm * (BM / 2) + 16 * i + 4 * (lane >> 4) + q;
            const int tok = row_token[r];
            float m = 0.0f;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                float zv = 0.0f;
                if (tok >= 0) {
                    int pg[L], pu[L];
#pragma unroll
                    for (int l = 0; l < L; ++l) {
                        const int ds = (zg | zu) ? xdsum[(int64_t)l * tokens + tok] : 0;
                        pg[l] = acc[i][j][l][q] - zg * ds;
                        pu[l] = acc[i][j + 2][l][q] - zu * ds;
                    }
                    const float sx = xscale[tok];
                    const float g = __fmul_rn(hm_recombine(pg, L), __fmul_rn(sx, sg));
                    const float u = __fmul_rn(hm_recombine(pu, L), __fmul_rn(sx, su));
                    zv = __fmul_rn(hm_silu(g), u);
                }
                z[i][j][q] = zv;
                m = fmaxf(m, fabsf(zv));
            }
#pragma unroll
            for (int s = 1; s < 16; s <<= 1) m = fmaxf(m, __shfl_xor(m, s, 64));
            if ((lane & 15) == 0) red[r][wn] = m;
        }
    }
    __syncthreads();
    const float range = (float)hm_limb_range(L);
    const int64_t nb = I / kZBlock;
    const int64_t zb = n0 / kZBlock;
#pragma unroll
    for (int i = 0; i < WM; ++i) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int r = wm * (BM / 2) + 16 * i + 4 * (lane >> 4) + q;
            const float amax = fmaxf(fmaxf(red[r][0], red[r][1]), fmaxf(red[r][2], red[r][3]));
            const float inv = amax > 0.0f ? __fdiv_rn(range, amax) : 0.0f;
            int dsum[L];
#pragma unroll
            for (int l = 0; l < L; ++l) dsum[l] = 0;
            if (r < nrows) {
                const int64_t grow = g0 + r;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int64_t col = n0 + 32 * wn + 16 * j + (lane & 15);
                    const int v = hm_fixed_point(z[i][j][q], inv, range);
#pragma unroll
                    for (int l = 0; l < L; ++l) {
                        const int d = hm_digit(v, l);
                        zdig[((int64_t)l * R + grow) * I + col] = (int8_t)d;
                        dsum[l] += d;
                    }
                }
                if (wn == 0 && (lane & 15) == 0) {
                    zscale[grow * nb + zb] = amax > 0.0f ? __fdiv_rn(amax, range) : 0.0f;
                }
            }
            if (zd != 0) {
#pragma unroll
                for (int l = 0; l < L; ++l) {
                    int s = dsum[l];
#pragma unroll
                    for (int sh = 1; sh < 16; sh <<= 1) s += __shfl_xor(s, sh, 64);
                    if ((lane & 15) == 0) red_i[l][r][wn] = s;
                }
            }
        }
    }
    if (zd != 0) {
        __syncthreads();
        if (tid < nrows) {
#pragma unroll
            for (int l = 0; l < L; ++l) {
                zdsum[((int64_t)l * R + g0 + tid) * nb + zb] =
                    red_i[l][tid][0] + red_i[l][tid][1] + red_i[l][tid][2] + red_i[l][tid][3];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// down: tile = BM contiguous grouped rows x 256 output columns; wave (wm, wn)
// owns rows [wm*BM/2, +BM/2) and columns [64 wn, 64 wn + 64).  At the end of
// each 128-column Z segment the exact partials are recombined and folded into
// the float accumulator: acc = fmaf(c, s_segment * scale_down, acc).
// ---------------------------------------------------------------------------
template <int L>
__global__ __launch_bounds__(kThreads) void down_mfma_kernel(
    const int8_t* __restrict__ zdig, const float* __restrict__ zscale,
    const int32_t* __restrict__ zdsum, int64_t R, int64_t H, int64_t I,
    int64_t experts, const int8_t* __restrict__ packed,
    const float* __restrict__ scale, const int32_t* __restrict__ zp,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    float* __restrict__ y) {
    constexpr int WM = Tiles<L>::WM, BM = Tiles<L>::BM;
    constexpr int A_CHUNKS = L * BM * 4;
    constexpr int NA = (A_CHUNKS + kThreads - 1) / kThreads;
    constexpr int MAXNB = 16;  // Z segments staged in LDS (I <= 2048)
    __shared__ __attribute__((aligned(16))) int8_t lds_a[2][L][BM][kRow];
    __shared__ __attribute__((aligned(16))) int8_t lds_b[2][256][kRow];
    __shared__ float s_alpha[MAXNB][BM];
    __shared__ int s_dsum[L][MAXNB][BM];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 2, wn = wave & 3;
    int64_t e, mt;
    if (!hm_locate_tile(counts, experts, BM, blockIdx.x, &e, &mt)) return;
    const int64_t g0 = offsets[e] + mt * BM;
    const int nrows = (int)min((int64_t)BM, (int64_t)counts[e] - mt * BM);
    const int64_t n0 = (int64_t)blockIdx.y * kDownN;
    const int nb = (int)(I / kZBlock);
    const float sd = scale[e * 3 + 2];
    const int zd = zp[e * 3 + 2];
    for (int i = tid; i < nb * BM; i += kThreads) {
        const int b = i / BM, r = i % BM;
        const int64_t grow = g0 + (r < nrows ? r : 0);
        s_alpha[b][r] = __fmul_rn(zscale[grow * nb + b], sd);
        for (int l = 0; l < L; ++l) s_dsum[l][b][r] = zd ? zdsum[((int64_t)l * R + grow) * nb + b] : 0;
    }

    const int8_t* dbase = packed + e * 3 * H * I + 2 * H * I;
    const int8_t* a_src[NA];
    int a_dst[NA];
#pragma unroll
    for (int c = 0; c < NA; ++c) {
        const int chunk = tid + c * kThreads;
        a_src[c] = nullptr;
        a_dst[c] = -1;
        if (chunk < A_CHUNKS) {
            const int l = chunk / (BM * 4), rem = chunk % (BM * 4);
            const int r = rem >> 2, seg = rem & 3;
            a_dst[c] = (l * BM + r) * kRow + 16 * seg;
            if (r < nrows) a_src[c] = zdig + ((int64_t)l * R + g0 + r) * I + 16 * seg;
        }
    }
    const int8_t* b_src[2];
    int b_dst[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int chunk = tid + c * kThreads;
        const int r = chunk >> 2, seg = chunk & 3;
        b_src[c] = dbase + (n0 + r) * I + 16 * seg;
        b_dst[c] = r * kRow + 16 * seg;
    }
    v4i ra[NA], rb[2];
    auto fetch = [&](int64_t k0) {
#pragma unroll
        for (int c = 0; c < NA; ++c) ra[c] = a_src[c] ? ld16(a_src[c] + k0) : v4i{0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < 2; ++c) rb[c] = ld16(b_src[c] + k0);
    };
    auto stash = [&](int buf) {
        int8_t* a = &lds_a[buf][0][0][0];
#pragma unroll
        for (int c = 0; c < NA; ++c) if (a_dst[c] >= 0) st16(a + a_dst[c], ra[c]);
        int8_t* b = &lds_b[buf][0][0];
#pragma unroll
        for (int c = 0; c < 2; ++c) st16(b + b_dst[c], rb[c]);
    };

    v4i acc[WM][4][L];
    float facc[WM][4][4];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int l = 0; l < L; ++l) acc[i][j][l] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int q = 0; q < 4; ++q) facc[i][j][q] = 0.0f;
        }

    const int nk = (int)(I / kStepK);
    fetch(0);
    stash(0);
    __syncthreads();
    const int arow = wm * (BM / 2) + (lane & 15);
    const int kofs = 16 * (lane >> 4);
    for (int ks = 0; ks < nk; ++ks) {
        const int buf = ks & 1;
        if (ks + 1 < nk) fetch((int64_t)(ks + 1) * kStepK);
        v4i b[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j] = ld16(&lds_b[buf][64 * wn + 16 * j + (lane & 15)][kofs]);
#pragma unroll
        for (int i = 0; i < WM; ++i) {
#pragma unroll
            for (int l = 0; l < L; ++l) {
                const v4i a = ld16(&lds_a[buf][l][arow + 16 * i][kofs]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[i][j][l] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[j], acc[i][j][l], 0, 0, 0);
                }
            }
        }
        if (ks & 1) {  // end of a 128-column Z segment (two 64-wide steps)
            const int zb = ks >> 1;
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int r = wm * (BM / 2) + 16 * i + 4 * (lane >> 4) + q;
                    const float alpha = s_alpha[zb][r];
                    int ds[L];
#pragma unroll
                    for (int l = 0; l < L; ++l) ds[l] = s_dsum[l][zb][r];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        int p[L];
#pragma unroll
                        for (int l = 0; l < L; ++l) {
                            p[l] = acc[i][j][l][q] - zd * ds[l];
                            acc[i][j][l][q] = 0;
                        }
                        facc[i][j][q] = __builtin_fmaf(hm_recombine(p, L), alpha, facc[i][j][q]);
                    }
                }
        }
        if (ks + 1 < nk) stash(buf ^ 1);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int r = wm * (BM / 2) + 16 * i + 4 * (lane >> 4) + q;
            if (r >= nrows) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t col = n0 + 64 * wn + 16 * j + (lane & 15);
                y[(g0 + r) * H + col] = facc[i][j][q];
            }
        }
}

}  // namespace

// Shape preconditions of the MFMA kernels (checked by the caller):
// H % 256 == 0, I % 128 == 0, I <= 2048.
bool hm_mfma_shape_ok(int64_t H, int64_t I) {
    return H % kDownN == 0 && I % kGateUpN == 0 && I % kZBlock == 0 && I / kZBlock <= 16;
}

int64_t hm_max_tiles(int64_t pairs, int64_t experts, int64_t tile_m);

template <int L>
static int launch_gateup(const hm_layer* layer, const int8_t* xdig, const float* xscale,
                         const int32_t* xdsum, int64_t tokens, const int32_t* counts,
                         const int32_t* offsets, const int32_t* perm_tokens, int64_t R,
                         int8_t* zdig, float* zscale, int32_t* zdsum, hipStream_t stream) {
    const int64_t H = layer->hidden, I = layer->intermediate, E = layer->experts;
    const dim3 grid((unsigned)hm_max_tiles(R, E, Tiles<L>::BM), (unsigned)(I / kGateUpN));
    hipLaunchKernelGGL(gateup_mfma_kernel<L>, grid, dim3(kThreads), 0, stream, xdig, xscale,
                       xdsum, tokens, H, I, E, static_cast<const int8_t*>(layer->packed),
                       layer->scale, layer->zero_point, counts, offsets, perm_tokens, R, zdig,
                       zscale, zdsum);
    HM_LAUNCHED();
    return HM_OK;
}

template <int L>
static int launch_down(const hm_layer* layer, const int32_t* counts, const int32_t* offsets,
                       int64_t R, const int8_t* zdig, const float* zscale,
                       const int32_t* zdsum, float* y, hipStream_t stream) {
    const int64_t H = layer->hidden, I = layer->intermediate, E = layer->experts;
    const dim3 grid((unsigned)hm_max_tiles(R, E, Tiles<L>::BM), (unsigned)(H / kDownN));
    hipLaunchKernelGGL(down_mfma_kernel<L>, grid, dim3(kThreads), 0, stream, zdig, zscale,
                       zdsum, R, H, I, E, static_cast<const int8_t*>(layer->packed),
                       layer->scale, layer->zero_point, counts, offsets, y);
    HM_LAUNCHED();
    return HM_OK;
}

int hm_launch_gateup_i8_mfma(const hm_layer* layer, int32_t limbs, const int8_t* xdig,
                             const float* xscale, const int32_t* xdsum, int64_t tokens,
                             const int32_t* counts, const int32_t* offsets,
                             const int32_t* perm_tokens, int64_t R, int8_t* zdig,
                             float* zscale, int32_t* zdsum, hipStream_t stream) {
    switch (limbs) {
    case 1: return launch_gateup<1>(layer, xdig, xscale, xdsum, tokens, counts, offsets, perm_tokens, R, zdig, zscale, zdsum, stream);
    case 2: return launch_gateup<2>(layer, xdig, xscale, xdsum, tokens, counts, offsets, perm_tokens, R, zdig, zscale, zdsum, stream);
    case 3: return launch_gateup<3>(layer, xdig, xscale, xdsum, tokens, counts, offsets, perm_tokens, R, zdig, zscale, zdsum, stream);
    default: return HM_ERR_INVALID;
    }
}

int hm_launch_down_i8_mfma(const hm_layer* layer, int32_t limbs, const int32_t* counts,
                           const int32_t* offsets, int64_t R, const int8_t* zdig,
                           const float* zscale, const int32_t* zdsum, float* y,
                           hipStream_t stream) {
    switch (limbs) {
    case 1: return launch_down<1>(layer, counts, offsets, R, zdig, zscale, zdsum, y, stream);
    case 2: return launch_down<2>(layer, counts, offsets, R, zdig, zscale, zdsum, y, stream);
    case 3: return launch_down<3>(layer, counts, offsets, R, zdig, zscale, zdsum, y, stream);
    default: return HM_ERR_INVALID;
    }
}
