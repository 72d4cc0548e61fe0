// hm_gemm_mfma.hip -- grouped INT8-MFMA expert GEMMs for gfx950.
//
// Both kernels run 512-thread workgroups (8 wave64s) over one tile of one
// expert's grouped rows.  The activation operand is L fixed-point digit
// planes (hm_device.h); every digit plane meets the same weight fragment in
// one v_mfma_i32_16x16x64_i8, so the int32 partial of each plane is exact.
//
// MFMA operand layout (v_mfma_i32_16x16x64_i8): lane l supplies 16 bytes of
// row (l % 16) of A and of column (l % 16) of B, K bytes 16*(l/16) ..
// 16*(l/16)+15 of the 64-wide step in both operands; the 4 int32 results of
// lane l are rows 4*(l/16) + 0..3 of column l % 16.
//
// Data movement: operands go straight from global memory to LDS with the
// gfx950 16-byte global_load_lds (lane l's 16 bytes land at base + 16*l)
// into fragments of 16 rows x KB bytes (KB = 128 for gate/up: every row load
// is a full 128-byte line; 64 for down) in a swizzled order that keeps both
// the global reads coalesced per row and the MFMA's ds_read_b128 bank-
// conflict free (Frag), and no registers stage the data.  A ring of S stages
// keeps S-1 K steps of loads in flight; one s_waitcnt vmcnt + barrier per
// step.  The K loop is unrolled by S so that every step reads and fills
// distinct LDS arrays.
//
// Tile order: the grid is 1D; workgroup i runs on XCD i % 8 (round-robin
// dispatch), so the linear tile index is remapped to give each XCD a
// contiguous run of (m-tile major, n-block minor) tiles: the n-blocks of an
// m-tile share its gathered activation rows, consecutive m-tiles of one
// expert share its weight columns, all in one XCD's L2.
#include "hm_device.h"
#include "hm_lds_dma.h"

#include <limits.h>

namespace {

constexpr int kThreads = 512;
constexpr int kWaves = 8;
constexpr int kMfmaK = 64;          // K bytes of one v_mfma_i32_16x16x64_i8
constexpr int kZBlock = 128;
constexpr int kGateUpN = 128;       // columns per projection per gate/up tile
constexpr int kDownN = 512;         // output columns per down tile (16 * Tile<L,true>::BFRAGS)
constexpr int kXcds = 8;

typedef int v4i __attribute__((ext_vector_type(4)));

// Fragment layout in LDS.  The wave-wide load that fills a fragment gives
// lane l row l/4 and 16-byte K chunk (l%4) ^ ((l/16)%4) of the 16 x 64 byte
// block: four adjacent lanes read one row's 64 contiguous bytes (one request
// per row instead of one per lane).  The MFMA reader lane m (row m%16, chunk
// m/16) finds its bytes at 16*(4*row + (chunk ^ (row/4))); over any 16
// consecutive reader lanes these are 16 distinct 16-byte bank groups, so the
// ds_read_b128 stays conflict free.
//
// With 128 K bytes per ring step a fragment is 16 rows x 128 bytes, two
// wave-wide loads (rows 0-7, 8-15): lane l takes row 8i + l/8 and 16-byte
// chunk (l%8) ^ ((row/2)%8), so 8 lanes read one row's full 128-byte line;
// reader lane m of K half h (row m%16, chunk 4h + m/16) finds its bytes at
// 1024*(row/8) + 16*(8*(row%8) + (chunk ^ (row/2)%8)), again 16 distinct
// bank groups over any 16 consecutive lanes.
template <int KB>
struct Frag {
    static constexpr int BYTES = 16 * KB;   // 16 rows of KB bytes
    static constexpr int LOADS = KB / 64;   // 1 KB wave-wide loads per fragment
    static constexpr int SUB = KB / kMfmaK; // MFMA K steps per ring step
    static_assert(KB == 64 || KB == 128, "fragment K width");
    // row (0..15) and 16-byte chunk loaded by `lane` in load i
    __device__ static int load_row(int lane, int i) {
        return KB == 64 ? lane >> 2 : 8 * i + (lane >> 3);
    }
    __device__ static int load_chunk(int lane, int i) {
        if (KB == 64) return (lane & 3) ^ ((lane >> 4) & 3);
        const int r = load_row(lane, i);
        return (lane & 7) ^ ((r >> 1) & 7);
    }
    // byte offset read by MFMA lane m in K step h of the fragment
    __device__ static int read_offset(int m, int h) {
        const int r = m & 15, c = 4 * h + (m >> 4);
        if (KB == 64) return 16 * (4 * r + (c ^ (r >> 2)));
        return 1024 * (r >> 3) + 16 * (8 * (r & 7) + (c ^ ((r >> 1) & 7)));
    }
};

// Tile traits: WM 16-row subtiles per wave, two row groups of waves.
// gate/up: wave = WM*16 rows (WM = 4, or 2 at three limbs) x (2 gate + 2 up)
// 16-column fragments, tile 2*WM*16 rows x 256 weight rows.  down: wave =
// WM*16 rows x 8 fragments (128
// columns), tile 2*WM*16 rows x 512 columns.  A wave's (WM*L) A fragments
// times its JB B fragments give MFMAs that each need 384 LDS bytes or
// fewer (8 A x 4 B, 4 A x 8 B), within the LDS bandwidth at full MFMA rate.
template <int L, bool DOWN>
struct Tile {
    static constexpr int WM = DOWN ? (L >= 3 ? 1 : 2) : (L >= 3 ? 2 : 4);  // 16-row subtiles per wave
    static constexpr int JB = DOWN ? 8 : 4;                   // B fragments per wave
    static constexpr int BM = 2 * 16 * WM;
    static constexpr int BFRAGS = 4 * JB;                     // B fragments per tile
    static constexpr int NA = L * BM / 16;                    // A fragments / stage
    static constexpr int NF = NA + BFRAGS;                    // fragments / stage
    static constexpr int KB = DOWN ? 64 : 128;                // K bytes per ring step
    using F = Frag<KB>;
    static constexpr int NL = NF * F::LOADS;                  // wave loads / stage
    static constexpr int LPW = (NL + kWaves - 1) / kWaves;    // loads per wave / stage
    // ring depth: as many stages as fit in ~136 KB of LDS, at least 2
    static constexpr int S = NF * F::BYTES * 4 <= 139264 ? 4
                           : NF * F::BYTES * 3 <= 139264 ? 3 : 2;
    static constexpr int STAGE_BYTES = NF * F::BYTES;
};

__device__ __forceinline__ v4i lds16(const int8_t* p) {
    return *reinterpret_cast<const v4i*>(p);
}



// The K loop over nk steps with a ring of S LDS stages.  Stage ks lives in
// ring (ks % S); step ks waits until at most S-2 later stages of this wave's
// loads are outstanding, meets the other waves at the barrier (after which
// every wave's loads of stage ks have landed and every read of the slot
// refilled next is done), refills that slot with step ks+S-1 and computes
// stage ks.  The steady state, where every step refills, runs unguarded; the
// last steps drain the ring.  The stages are distinct arrays named at compile
// time in every unrolled step.
template <int S, int LPW, int KB, class Issue, class Compute>
__device__ __forceinline__ void ring_loop(int nk, int8_t* r0, int8_t* r1, int8_t* r2, int8_t* r3,
                                          Issue&& issue, Compute&& compute) {
    auto slot = [&](int s) -> int8_t* {
        return s == 0 ? r0 : s == 1 ? r1 : s == 2 ? r2 : r3;
    };
#pragma unroll
    for (int s = 0; s < S - 1; ++s) {
        if (s < nk) issue(slot(s), (int64_t)s * KB);
    }
    int ks0 = 0;
    for (; ks0 + 2 * S - 2 < nk; ks0 += S) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            wait_vmcnt<(S - 2) * LPW>();
            lds_barrier();
            issue(slot((s + S - 1) % S), (int64_t)(ks0 + s + S - 1) * KB);
            compute(slot(s), ks0 + s);
        }
    }
    for (; ks0 < nk; ks0 += S) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int ks = ks0 + s;
            if (ks < nk) {
                if (ks + S - 2 < nk) wait_vmcnt<(S - 2) * LPW>();
                else wait_vmcnt<0>();
                lds_barrier();
                if (ks + S - 1 < nk) issue(slot((s + S - 1) % S), (int64_t)(ks + S - 1) * KB);
                compute(slot(s), ks);
            }
        }
    }
}

// Linear workgroup -> logical tile (m-tile major, n-block minor), grouped
// per XCD.  Returns false for the padding workgroups of the last XCD.
__device__ __forceinline__ bool xcd_tile(int64_t mtiles, int64_t nblocks, int64_t* mt,
                                         int64_t* nb) {
    const int64_t total = mtiles * nblocks;
    const int64_t per = (total + kXcds - 1) / kXcds;
    const int64_t i = blockIdx.x;
    const int64_t j = (i % kXcds) * per + i / kXcds;
    if (j >= total) return false;
    *mt = j / nblocks;
    *nb = j % nblocks;
    return true;
}

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
    int64_t experts, int64_t mtiles, const int8_t* __restrict__ packed,
    const float* __restrict__ scale, const int32_t* __restrict__ zp,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ perm_tokens, int64_t R, int8_t* __restrict__ zdig,
    float* __restrict__ zscale, int32_t* __restrict__ zdsum) {
    using T = Tile<L, false>;
    using F = typename T::F;
    constexpr int WM = T::WM, BM = T::BM, NA = T::NA, NL = T::NL, LPW = T::LPW, S = T::S,
                  KB = T::KB;
    __shared__ __attribute__((aligned(1024))) int8_t ring0[T::STAGE_BYTES];
    __shared__ __attribute__((aligned(1024))) int8_t ring1[T::STAGE_BYTES];
    __shared__ __attribute__((aligned(1024))) int8_t ring2[T::STAGE_BYTES];
    __shared__ __attribute__((aligned(1024))) int8_t ring3[S > 3 ? T::STAGE_BYTES : 16];
    __shared__ int32_t row_token[BM];
    __shared__ unsigned long long s_exp2[32];
    __shared__ float s_xscale[BM];
    __shared__ int32_t s_xdsum[L][BM];
    __shared__ float red[BM][4];
    __shared__ int red_i[L][BM][4];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 2, wn = wave & 3;
    int rd[F::SUB];
#pragma unroll
    for (int h = 0; h < F::SUB; ++h) rd[h] = F::read_offset(lane, h);
    int64_t gmt, nb;
    if (!xcd_tile(mtiles, I / kGateUpN, &gmt, &nb)) return;
    int64_t e, mt;
    if (!hm_locate_tile(counts, experts, BM, gmt, &e, &mt)) return;
    const int64_t g0 = offsets[e] + mt * BM;
    const int nrows = (int)min((int64_t)BM, (int64_t)counts[e] - mt * BM);
    const int64_t n0 = nb * kGateUpN;
    if (tid < BM) row_token[tid] = perm_tokens[g0 + (tid < nrows ? tid : 0)];
    hm_load_exp2_table(s_exp2);
    __syncthreads();
    // per-row activation scale (and digit sums if a zero point needs them)
    // for the epilogue, fetched while the K loop runs
    const int zg = zp[e * 3 + 0], zu = zp[e * 3 + 1];
    if (tid < BM) {
        const int tok = row_token[tid];
        s_xscale[tid] = xscale[tok];
#pragma unroll
        for (int l = 0; l < L; ++l) s_xdsum[l][tid] = (zg | zu) ? xdsum[(int64_t)l * tokens + tok] : 0;
    }

    // Per-lane global source of each fragment this wave loads (K offset 0).
    const int8_t* ebase = packed + e * 3 * H * I;
    const int8_t* src[LPW];
    int dst[LPW];
#pragma unroll
    for (int c = 0; c < LPW; ++c) {
        const int u = (wave + kWaves * c) % NL;   // load unit: fragment f, part li
        const int f = u / F::LOADS, li = u % F::LOADS;
        const int fr = F::load_row(lane, li), ch = F::load_chunk(lane, li);
        dst[c] = f * F::BYTES + 1024 * li;
        if (f < NA) {
            const int l = f / (BM / 16), i = f % (BM / 16);
            const int tok = row_token[16 * i + fr];
            src[c] = xdig + ((int64_t)l * tokens + tok) * H + 16 * ch;
        } else {
            const int brow = 16 * (f - NA) + fr;
            const int64_t col = n0 + (brow & 127);
            src[c] = ebase + (brow >> 7) * H * I + col * H + 16 * ch;
        }
    }
    auto issue = [&](int8_t* stage, int64_t k0) {
#pragma unroll
        for (int c = 0; c < LPW; ++c) dma16(src[c] + k0, stage + dst[c]);  // wave-uniform base
    };

    v4i acc[WM][4][L];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int l = 0; l < L; ++l) acc[i][j][l] = v4i{0, 0, 0, 0};

    auto compute = [&](const int8_t* stage) {
#pragma unroll
        for (int h = 0; h < F::SUB; ++h) {
            v4i b[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int bf = (j >> 1) * 8 + 2 * wn + (j & 1);  // 16-row fragment index
                b[j] = lds16(stage + (NA + bf) * F::BYTES + rd[h]);
            }
#pragma unroll
            for (int i = 0; i < WM; ++i) {
#pragma unroll
                for (int l = 0; l < L; ++l) {
                    const v4i a = lds16(stage + (l * (BM / 16) + wm * WM + i) * F::BYTES + rd[h]);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        acc[i][j][l] =
                            __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[j], acc[i][j][l], 0, 0, 0);
                    }
                }
            }
        }
    };

    ring_loop<S, LPW, KB>((int)(H / KB), ring0, ring1, ring2, ring3, issue,
                      [&](const int8_t* stage, int) { compute(stage); });

    // ---- epilogue -------------------------------------------------------
    const float sg = scale[e * 3 + 0], su = scale[e * 3 + 1];
    const int zd = zp[e * 3 + 2];
    float z[WM][2][4];
    // every row is computed (rows past nrows repeat row 0's token and are
    // zeroed at the end), so the epilogue runs without divergence
#pragma unroll
    for (int i = 0; i < WM; ++i) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int r = wm * (BM / 2) + 16 * i + 4 * (lane >> 4) + q;
            const bool live = r < nrows;
            const float sx = s_xscale[r];
            const float fg = __fmul_rn(sx, sg), fu = __fmul_rn(sx, su);
            int ds[L];
#pragma unroll
            for (int l = 0; l < L; ++l) ds[l] = s_xdsum[l][r];   // zeros without zero points
            float m = 0.0f;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                int pg[L], pu[L];
#pragma unroll
                for (int l = 0; l < L; ++l) {
                    pg[l] = acc[i][j][l][q] - zg * ds[l];
                    pu[l] = acc[i][j + 2][l][q] - zu * ds[l];
                }
                const float g = __fmul_rn(hm_recombine(pg, L), fg);
                const float u = __fmul_rn(hm_recombine(pu, L), fu);
                float sv = hm_silu_t(g, s_exp2);
                asm volatile("" : "+v"(sv));  // computed on every lane: no branch
                const float zv = live ? __fmul_rn(sv, u) : 0.0f;
                z[i][j][q] = zv;
                m = fmaxf(m, fabsf(zv));
            }
            m = hm_row16_max(m);
            if ((lane & 15) == 0) red[r][wn] = m;
        }
    }
    __syncthreads();
    const float range = (float)hm_limb_range(L);
    const int64_t nbz = I / kZBlock;
    const int64_t zb = n0 / kZBlock;
    // the digits of the tile's Z segment: [L][BM][128] bytes (staged in LDS,
    // stored below with 16-byte writes)
    int zfix[WM][2][4];
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
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int v = hm_fixed_point(z[i][j][q], inv, range);
                zfix[i][j][q] = v;
#pragma unroll
                for (int l = 0; l < L; ++l) dsum[l] += hm_digit(v, l);
            }
            if (r < nrows && wn == 0 && (lane & 15) == 0) {
                zscale[(g0 + r) * nbz + zb] = amax > 0.0f ? __fdiv_rn(amax, range) : 0.0f;
            }
            if (zd != 0) {
#pragma unroll
                for (int l = 0; l < L; ++l) {
                    const int s = hm_row16_sum(dsum[l]);
                    if ((lane & 15) == 0) red_i[l][r][wn] = s;
                }
            }
        }
    }
    // digit planes out through LDS (ring0, free after the K loop): byte
    // writes into [BM][128], then 16-byte rows segments to zdig
    int8_t* zst = ring0;
#pragma unroll
    for (int l = 0; l < L; ++l) {
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int r = wm * (BM / 2) + 16 * i + 4 * (lane >> 4) + q;
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    zst[r * kGateUpN + 32 * wn + 16 * j + (lane & 15)] = (int8_t)hm_digit(zfix[i][j][q], l);
            }
        __syncthreads();
        for (int c = tid; c < nrows * (kGateUpN / 16); c += kThreads) {
            const int r = c / (kGateUpN / 16), c16 = c % (kGateUpN / 16);
            const int4 v = *reinterpret_cast<const int4*>(zst + r * kGateUpN + 16 * c16);
            *reinterpret_cast<int4*>(zdig + ((int64_t)l * R + g0 + r) * I + n0 + 16 * c16) = v;
        }
        __syncthreads();
    }
    if (zd != 0) {
        if (tid < nrows) {
#pragma unroll
            for (int l = 0; l < L; ++l) {
                zdsum[((int64_t)l * R + g0 + tid) * nbz + zb] =
                    red_i[l][tid][0] + red_i[l][tid][1] + red_i[l][tid][2] + red_i[l][tid][3];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// down: tile = BM contiguous grouped rows x 512 output columns; wave (wm, wn)
// owns rows [wm*BM/2, +BM/2) and columns [128 wn, 128 wn + 128).  At the end of
// each 128-column Z segment the exact partials are recombined and folded into
// the float accumulator: acc = fmaf(c, s_segment * scale_down, acc).
// ---------------------------------------------------------------------------
template <int L>
__global__ __launch_bounds__(kThreads) void down_mfma_kernel(
    const int8_t* __restrict__ zdig, const float* __restrict__ zscale,
    const int32_t* __restrict__ zdsum, int64_t R, int64_t H, int64_t I,
    int64_t experts, int64_t mtiles, const int8_t* __restrict__ packed,
    const float* __restrict__ scale, const int32_t* __restrict__ zp,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    float* __restrict__ y) {
    using T = Tile<L, true>;
    using F = typename T::F;
    constexpr int WM = T::WM, JB = T::JB, BM = T::BM, NA = T::NA, NL = T::NL, LPW = T::LPW,
                  S = T::S, KB = T::KB;
    constexpr int BN = 16 * T::BFRAGS;  // output columns per tile
    constexpr int MAXNB = 16;           // Z segments (I <= 2048)
    __shared__ __attribute__((aligned(1024))) int8_t ring0[T::STAGE_BYTES];
    __shared__ __attribute__((aligned(1024))) int8_t ring1[T::STAGE_BYTES];
    __shared__ __attribute__((aligned(1024))) int8_t ring2[T::STAGE_BYTES];
    __shared__ __attribute__((aligned(1024))) int8_t ring3[S > 3 ? T::STAGE_BYTES : 16];
    __shared__ float s_alpha[MAXNB][BM];
    __shared__ int32_t s_corr[MAXNB][L][BM];  // zp * digit sum of each Z segment

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 2, wn = wave & 3;
    int rd[F::SUB];
#pragma unroll
    for (int h = 0; h < F::SUB; ++h) rd[h] = F::read_offset(lane, h);
    int64_t gmt, nb;
    if (!xcd_tile(mtiles, H / BN, &gmt, &nb)) return;
    int64_t e, mt;
    if (!hm_locate_tile(counts, experts, BM, gmt, &e, &mt)) return;
    const int64_t g0 = offsets[e] + mt * BM;
    const int nrows = (int)min((int64_t)BM, (int64_t)counts[e] - mt * BM);
    const int64_t n0 = nb * BN;
    const int nbz = (int)(I / kZBlock);
    const float sd = scale[e * 3 + 2];
    const int zd = zp[e * 3 + 2];
    for (int i = tid; i < nbz * BM; i += kThreads) {
        const int b = i / BM, r = i % BM;
        const int64_t g = g0 + (r < nrows ? r : 0);
        s_alpha[b][r] = __fmul_rn(zscale[g * nbz + b], sd);
#pragma unroll
        for (int l = 0; l < L; ++l) s_corr[b][l][r] = zd ? zd * zdsum[((int64_t)l * R + g) * nbz + b] : 0;
    }

    const int8_t* dbase = packed + e * 3 * H * I + 2 * H * I;
    const int8_t* src[LPW];
    int dst[LPW];
#pragma unroll
    for (int c = 0; c < LPW; ++c) {
        const int u = (wave + kWaves * c) % NL;   // load unit: fragment f, part li
        const int f = u / F::LOADS, li = u % F::LOADS;
        const int fr = F::load_row(lane, li), ch = F::load_chunk(lane, li);
        dst[c] = f * F::BYTES + 1024 * li;
        if (f < NA) {
            const int l = f / (BM / 16), i = f % (BM / 16);
            const int r = 16 * i + fr;
            src[c] = zdig + ((int64_t)l * R + g0 + (r < nrows ? r : 0)) * I + 16 * ch;
        } else {
            const int brow = 16 * (f - NA) + fr;
            src[c] = dbase + (n0 + brow) * I + 16 * ch;
        }
    }
    auto issue = [&](int8_t* stage, int64_t k0) {
#pragma unroll
        for (int c = 0; c < LPW; ++c) dma16(src[c] + k0, stage + dst[c]);  // wave-uniform base
    };

    v4i acc[WM][JB][L];
    float facc[WM][JB][4];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < JB; ++j) {
#pragma unroll
            for (int l = 0; l < L; ++l) acc[i][j][l] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int q = 0; q < 4; ++q) facc[i][j][q] = 0.0f;
        }

    // The WM*L A fragments stay in registers while the JB weight fragments
    // stream through one register quad each (fewer live VGPRs than holding B).
    auto compute = [&](const int8_t* stage) {
#pragma unroll
        for (int h = 0; h < F::SUB; ++h) {
            v4i a[WM][L];
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int l = 0; l < L; ++l)
                    a[i][l] = lds16(stage + (l * (BM / 16) + wm * WM + i) * F::BYTES + rd[h]);
#pragma unroll
            for (int j = 0; j < JB; ++j) {
                const v4i b = lds16(stage + (NA + JB * wn + j) * F::BYTES + rd[h]);
#pragma unroll
                for (int i = 0; i < WM; ++i)
#pragma unroll
                    for (int l = 0; l < L; ++l)
                        acc[i][j][l] =
                            __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i][l], b, acc[i][j][l], 0, 0, 0);
            }
        }
    };
    auto fold = [&](int zb) {  // end of Z segment zb: exact partials -> float
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int r = wm * (BM / 2) + 16 * i + 4 * (lane >> 4) + q;
                const float alpha = s_alpha[zb][r];
                int ds[L];
#pragma unroll
                for (int l = 0; l < L; ++l) ds[l] = s_corr[zb][l][r];
#pragma unroll
                for (int j = 0; j < JB; ++j) {
                    int p[L];
#pragma unroll
                    for (int l = 0; l < L; ++l) {
                        p[l] = acc[i][j][l][q] - ds[l];
                        acc[i][j][l][q] = 0;
                    }
                    facc[i][j][q] = __builtin_fmaf(hm_recombine(p, L), alpha, facc[i][j][q]);
                }
            }
    };

    __syncthreads();  // s_alpha, s_corr visible (before any LDS DMA is in flight)
    static_assert(kZBlock % KB == 0, "a ring step never straddles a Z segment");
    constexpr int kStepsPerSeg = kZBlock / KB;
    ring_loop<S, LPW, KB>((int)(I / KB), ring0, ring1, ring2, ring3, issue,
                      [&](const int8_t* stage, int ks) {
                          compute(stage);
                          if (ks % kStepsPerSeg == kStepsPerSeg - 1) fold(ks / kStepsPerSeg);
                      });
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int r = wm * (BM / 2) + 16 * i + 4 * (lane >> 4) + q;
            if (r >= nrows) continue;
#pragma unroll
            for (int j = 0; j < JB; ++j) {
                const int64_t col = n0 + 16 * (JB * wn + j) + (lane & 15);
                y[(g0 + r) * H + col] = facc[i][j][q];
            }
        }
}

}  // namespace

// Shape preconditions of the MFMA kernels (checked by the caller):
// H % 256 == 0, I % 128 == 0, I <= 2048.
static_assert(16 * Tile<2, true>::BFRAGS == kDownN && 16 * Tile<3, true>::BFRAGS == kDownN, "down tile width");

bool hm_mfma_shape_ok(int64_t H, int64_t I) {
    return H % kDownN == 0 && I % kGateUpN == 0 && I % kZBlock == 0 && I / kZBlock <= 16;
}

int64_t hm_max_tiles(int64_t pairs, int64_t experts, int64_t tile_m);

static unsigned xcd_grid(int64_t mtiles, int64_t nblocks) {
    const int64_t total = mtiles * nblocks;
    return (unsigned)(((total + kXcds - 1) / kXcds) * kXcds);
}

template <int L>
static int launch_gateup(const hm_layer* layer, const int8_t* xdig, const float* xscale,
                         const int32_t* xdsum, int64_t tokens, const int32_t* counts,
                         const int32_t* offsets, const int32_t* perm_tokens, int64_t R,
                         int8_t* zdig, float* zscale, int32_t* zdsum, hipStream_t stream) {
    const int64_t H = layer->hidden, I = layer->intermediate, E = layer->experts;
    const int64_t mtiles = hm_max_tiles(R, E, Tile<L, false>::BM);
    hipLaunchKernelGGL(gateup_mfma_kernel<L>, dim3(xcd_grid(mtiles, I / kGateUpN)),
                       dim3(kThreads), 0, stream, xdig, xscale, xdsum, tokens, H, I, E, mtiles,
                       static_cast<const int8_t*>(layer->packed), layer->scale,
                       layer->zero_point, counts, offsets, perm_tokens, R, zdig, zscale, zdsum);
    HM_LAUNCHED();
    return HM_OK;
}

template <int L>
static int launch_down(const hm_layer* layer, const int32_t* counts, const int32_t* offsets,
                       int64_t R, const int8_t* zdig, const float* zscale,
                       const int32_t* zdsum, float* y, hipStream_t stream) {
    const int64_t H = layer->hidden, I = layer->intermediate, E = layer->experts;
    const int64_t mtiles = hm_max_tiles(R, E, Tile<L, true>::BM);
    hipLaunchKernelGGL(down_mfma_kernel<L>, dim3(xcd_grid(mtiles, H / kDownN)), dim3(kThreads),
                       0, stream, zdig, zscale, zdsum, R, H, I, E, mtiles,
                       static_cast<const int8_t*>(layer->packed), layer->scale,
                       layer->zero_point, counts, offsets, y);
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
