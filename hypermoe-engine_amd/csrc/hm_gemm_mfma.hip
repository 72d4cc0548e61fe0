// hm_gemm_mfma.hip -- grouped INT8-MFMA expert GEMMs for gfx950.
//
// Both kernels are persistent: one 512-thread workgroup (8 wave64s, two per
// SIMD) per CU walks a list of output tiles of the grouped problem.  The
// activation operand is L fixed-point digit planes (hm_device.h); every digit plane
// meets the same weight fragment in one v_mfma_i32_32x32x32_i8, so the
// int32 partial of each plane is exact.
//
// MFMA operand layout (v_mfma_i32_32x32x32_i8): lane l supplies 16 bytes of
// row (l % 32) of A and of column (l % 32) of B, K bytes 16*(l/32) ..
// 16*(l/32)+15 of the 32-wide step; the 16 int32 results of lane l are
// column l % 32, rows 8*(v/4) + 4*(l/32) + v%4 for v = 0..15.  (The
// 16x16x64 form issues at half this rate on gfx950 unless a wave keeps many
// more independent accumulators in flight.)
//
// Data movement: operands go straight from global memory to LDS with the
// 16-byte global_load_lds (lane l's 16 bytes land at base + 16*l) into
// fragments of 32 rows x 64 K bytes, swizzled so that the global reads stay
// coalesced per row and the MFMA's ds_read_b128 stays bank-conflict free.
// A ring of kS stages (64 K bytes each) keeps kS-1 stages in flight; the
// fragments of stage ks+1 are read into registers while the MFMAs of stage
// ks run, so a stage's LDS slot is free for refill one step after it lands.
//
// Tile stream: each workgroup's tiles form one stream of K stages.  The
// first kS-1 stages of the next tile are issued while the current tile
// finishes, and its per-row metadata (token ids, scales) is fetched into a
// second LDS buffer by the same in-order DMA queue, so the epilogue of a
// tile runs while the next tile's operands are already landing.  All global
// loads inside the stream are LDS DMA: the compiler's own waits for a
// register load would otherwise drain the queue.
//
// Tile order: the real tile count comes from the routed counts on the
// device.  Tiles are numbered m-tile major, n-block minor and split into 8
// contiguous ranges, one per XCD (workgroup i runs on XCD i % 8), so the
// n-blocks of an m-tile (sharing its activation rows) and consecutive
// m-tiles of one expert (sharing its weight columns) meet in one XCD's L2.
#include "hm_device.h"
#include "hm_lds_dma.h"

#include <limits.h>

#include <type_traits>

namespace {

constexpr int kWaves = 8;           // wave64s per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kKB = 64;             // K bytes per ring stage: two 32-byte MFMA K steps
constexpr int kS = 4;               // ring stages (gate/up)
#ifndef HM_DOWN_STAGES
#define HM_DOWN_STAGES 5
#endif
// ring stages of the down projection (three limbs fill LDS at four)
template <int L>
constexpr int down_stages() { return L >= 3 ? 4 : HM_DOWN_STAGES; }
constexpr int kFragBytes = 32 * kKB;  // one 32-row fragment of a stage
constexpr int kZBlock = 128;        // Z fixed-point segment (columns of Z = K of down)
constexpr int kGateUpN = 128;       // columns per projection per gate/up tile
constexpr int kXcds = 8;
constexpr int kMaxExperts = 256;    // expert tables live in LDS
constexpr int kMaxZSeg = 6;         // down: Z segments per row held in LDS (I <= 768)

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// Fragment layout in LDS (32 rows x 64 bytes = two 1 KB halves of 16 rows).
// The wave-wide load that fills half hf gives lane l row 16*hf + l/4 and
// 16-byte K chunk (l%4) ^ ((l/16)%4): four adjacent lanes read one row's 64
// contiguous bytes.  The MFMA reader lane m of K step h (row r = m%32,
// chunk c = 2h + m/32) finds its bytes at
//   1024*(r/16) + 16*(4*(r%16) + (c ^ ((r/4)%4)))
// and over any 16 consecutive reader lanes these are 16 distinct 16-byte
// bank groups.
__device__ __forceinline__ int frag_load_row(int lane, int hf) { return 16 * hf + (lane >> 2); }
__device__ __forceinline__ int frag_load_chunk(int lane) { return (lane & 3) ^ ((lane >> 4) & 3); }
__device__ __forceinline__ int frag_read_offset(int lane, int h) {
    const int r = lane & 31, c = 2 * h + (lane >> 5);
    return 1024 * (r >> 4) + 16 * (4 * (r & 15) + (c ^ ((r >> 2) & 3)));
}

__device__ __forceinline__ v4i lds16(const int8_t* p) {
    return *reinterpret_cast<const v4i*>(p);
}

__device__ __forceinline__ v16i mfma32(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// Exclusive prefix of the m-tiles of every expert (ceil(count / bm)) into
// prefix[0..E], prefix[E] = total.  One full wave.
__device__ __forceinline__ void tile_prefix(const int32_t* cnt, int E, int bm, int32_t* prefix) {
    const int lane = threadIdx.x & (HM_WAVE - 1);
    int base = 0;
    for (int c0 = 0; c0 < E; c0 += HM_WAVE) {
        const int e = c0 + lane;
        const int n = e < E ? (cnt[e] + bm - 1) / bm : 0;
        int incl = n;
#pragma unroll
        for (int sft = 1; sft < HM_WAVE; sft <<= 1) {
            const int o = __shfl_up(incl, sft, HM_WAVE);
            if (lane >= sft) incl += o;
        }
        if (e < E) prefix[e] = base + incl - n;
        base += __shfl(incl, HM_WAVE - 1, HM_WAVE);
    }
    if (lane == 0) prefix[E] = base;
}

// Expert owning global m-tile gm: the last expert whose first tile is <= gm
// (prefix is non-decreasing; experts with no tiles share their successor's
// start and are skipped).  Every lane of the wave must be active.
__device__ __forceinline__ int locate_expert(const int32_t* prefix, int E, int gm) {
    const int lane = threadIdx.x & (HM_WAVE - 1);
    int n = 0;
    for (int c0 = 0; c0 < E; c0 += HM_WAVE) {
        const int e = c0 + lane;
        n += __popcll(__ballot(e < E && prefix[e] <= gm));
    }
    return __builtin_amdgcn_readfirstlane(n - 1);
}

// The workgroup's share of the tile list: tiles jbeg, jbeg + step, ... < jend
// of the XCD range [x*per, (x+1)*per).
struct TileRange {
    int jbeg, jend, step, ntiles;
};
__device__ __forceinline__ TileRange tile_range(int total) {
    TileRange t;
    const int per = (total + kXcds - 1) / kXcds;
    const int x = blockIdx.x % kXcds;
    t.step = gridDim.x / kXcds;
    t.jbeg = x * per + blockIdx.x / kXcds;
    t.jend = min((x + 1) * per, total);
    t.ntiles = t.jbeg < t.jend ? (t.jend - t.jbeg + t.step - 1) / t.step : 0;
    return t;
}

// Tile row of accumulator element v of lane `lane` in the 32-row fragment
// starting at row r0.
__device__ __forceinline__ int acc_row(int r0, int lane, int v) {
    return r0 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
}

// ---------------------------------------------------------------------------
// gate/up: tile = BM grouped rows x (128 gate + 128 up) weight columns.
// wave (wr, wc): rows [32*WR*wr, +32*WR), gate and up columns
// [32*WCP*wc, +32*WCP) of the tile.  Epilogue: z = silu(g) * u; the tile's
// 128-column fixed-point segment of each Z row is quantised to L digits.
// ---------------------------------------------------------------------------
template <int L>
struct GateUpTile {
    static constexpr int WR = 1;                        // 32-row fragments per wave
    static constexpr int WCP = L >= 3 ? 1 : 2;          // gate (and up) fragments per wave
    static constexpr int NWC = kGateUpN / 32 / WCP;     // waves across the columns
    static constexpr int NWR = kWaves / NWC;            // waves across the rows
    static constexpr int BM = 32 * WR * NWR;            // 128 rows (64 at three limbs)
    static constexpr int NA = L * BM / 32;              // A fragments per stage
    static constexpr int NB = 2 * kGateUpN / 32;        // 8 B fragments (4 gate, 4 up)
    static constexpr int NF = NA + NB;
    static constexpr int NL = 2 * NF;                   // wave-wide loads per stage
    static constexpr int LPW = (NL + kWaves - 1) / kWaves;
    static constexpr int STAGE = NF * kFragBytes;
};

template <int L>
__global__ __launch_bounds__(kThreads) void gateup_mfma_kernel(
    const int8_t* __restrict__ xdig, const float* __restrict__ xscale,
    const int32_t* __restrict__ xdsum, int tokens, int H, int I, int experts,
    const int8_t* __restrict__ packed, const float* __restrict__ scale,
    const int32_t* __restrict__ zp, const int32_t* __restrict__ counts,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ perm_tokens, int R,
    float* __restrict__ gout, float* __restrict__ uout) {
    using T = GateUpTile<L>;
    constexpr int BM = T::BM, NA = T::NA, NL = T::NL, LPW = T::LPW, WR = T::WR, WCP = T::WCP,
                  NWC = T::NWC, STAGE = T::STAGE;
    constexpr int RW = BM / HM_WAVE;  // waves that move one value per tile row
    __shared__ __attribute__((aligned(1024))) int8_t ring[kS * STAGE];
    __shared__ int32_t s_prefix[kMaxExperts + 1];
    __shared__ int32_t s_off[kMaxExperts], s_cnt[kMaxExperts];
    __shared__ float s_sg[kMaxExperts], s_su[kMaxExperts];
    __shared__ int32_t s_zg[kMaxExperts], s_zu[kMaxExperts];
    __shared__ __attribute__((aligned(16))) int32_t s_rt[2][BM];     // token of each tile row
    __shared__ __attribute__((aligned(16))) float s_xs[2][BM];       // its activation scale
    __shared__ __attribute__((aligned(16))) int32_t s_xd[2][L][BM];  // its digit sums

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = wave / NWC, wc = wave % NWC;
    const int E = (int)experts;
    for (int e = tid; e < E; e += kThreads) {
        s_cnt[e] = counts[e];
        s_off[e] = offsets[e];
        s_sg[e] = scale[3 * e + 0];
        s_su[e] = scale[3 * e + 1];
        s_zg[e] = zp[3 * e + 0];
        s_zu[e] = zp[3 * e + 1];
    }
    __syncthreads();
    if (wave == 0) tile_prefix(s_cnt, E, BM, s_prefix);
    __syncthreads();
    const int nbn = I / kGateUpN;
    const TileRange tr = tile_range(s_prefix[E] * nbn);
    if (tr.ntiles == 0) return;
    const int nk = (int)(H / kKB);

    struct Info {
        int e, nrows, g0, n0;
    };
    auto info = [&](int i) __attribute__((always_inline)) {
        const int j = tr.jbeg + i * tr.step;
        const int gm = j / nbn;
        Info t;
        t.e = locate_expert(s_prefix, E, gm);
        const int mt = gm - s_prefix[t.e];
        t.g0 = s_off[t.e] + mt * BM;
        t.nrows = min(BM, s_cnt[t.e] - mt * BM);
        t.n0 = (j % nbn) * kGateUpN;
        return t;
    };
    // token ids of the tile rows (rows past nrows repeat the last row)
    auto fetch_rows = [&](const Info& t, int m) __attribute__((always_inline)) {
        if (wave < RW) {
            const int r = HM_WAVE * wave + lane;
            dma4(perm_tokens + t.g0 + min(r, t.nrows - 1), &s_rt[m][HM_WAVE * wave]);
        }
    };
    // activation scales and digit sums of those tokens (needs s_rt[m])
    auto fetch_row_meta = [&](int m) __attribute__((always_inline)) {
        if (wave < RW) {
            const int tok = s_rt[m][HM_WAVE * wave + lane];
            dma4(xscale + tok, &s_xs[m][HM_WAVE * wave]);
#pragma unroll
            for (int l = 0; l < L; ++l) dma4(xdsum + (int64_t)l * tokens + tok, &s_xd[m][l][HM_WAVE * wave]);
        }
    };
    int dst[LPW];
#pragma unroll
    for (int c = 0; c < LPW; ++c) {
        const int u = (wave + kWaves * c) % NL;   // load unit: fragment u/2, half u%2
        dst[c] = (u >> 1) * kFragBytes + 1024 * (u & 1);
    }
    auto make_src = [&](const Info& t, int m, const int8_t* (&src)[LPW]) {
        const int8_t* ebase = packed + (int64_t)t.e * 3 * H * I;
        const int ch = frag_load_chunk(lane);
#pragma unroll
        for (int c = 0; c < LPW; ++c) {
            const int u = (wave + kWaves * c) % NL;
            const int f = u >> 1, row = frag_load_row(lane, u & 1);
            if (f < NA) {
                const int l = f / (BM / 32), i = f % (BM / 32);
                const int tok = s_rt[m][32 * i + row];
                src[c] = xdig + ((int64_t)l * tokens + tok) * H + 16 * ch;
            } else {
                const int fb = f - NA;
                const int64_t col = t.n0 + 32 * (fb & 3) + row;
                src[c] = ebase + (int64_t)(fb >> 2) * H * I + col * H + 16 * ch;
            }
        }
    };
    auto issue = [&](int slot, const int8_t* const (&src)[LPW], int ks) {
        int8_t* st = ring + slot * STAGE;
#pragma unroll
        for (int c = 0; c < LPW; ++c) dma16(src[c] + (int64_t)ks * kKB, st + dst[c]);
    };

    int rd[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) rd[h] = frag_read_offset(lane, h);
    v4i fa[2][WR][L], fb[2][2 * WCP];
    auto read_frags = [&](int slot, int h) __attribute__((always_inline)) {
        const int8_t* st = ring + slot * STAGE;
#pragma unroll
        for (int ii = 0; ii < WR; ++ii)
#pragma unroll
            for (int l = 0; l < L; ++l)
                fa[h][ii][l] = lds16(st + (l * (BM / 32) + wr * WR + ii) * kFragBytes + rd[h]);
#pragma unroll
        for (int j = 0; j < 2 * WCP; ++j) {
            const int fbi = j < WCP ? wc * WCP + j : 4 + wc * WCP + (j - WCP);
            fb[h][j] = lds16(st + (NA + fbi) * kFragBytes + rd[h]);
        }
    };
    v16i acc[WR][L][2 * WCP];
    // `first`: the tile's first K step starts the accumulators from zero
    auto mfma_step = [&](int h, auto first) __attribute__((always_inline)) {
#pragma unroll
        for (int ii = 0; ii < WR; ++ii)
#pragma unroll
            for (int l = 0; l < L; ++l)
#pragma unroll
                for (int j = 0; j < 2 * WCP; ++j) {
                    if constexpr (decltype(first)::value)
                        acc[ii][l][j] = mfma32(fa[h][ii][l], fb[h][j], v16i{});
                    else
                        acc[ii][l][j] = mfma32(fa[h][ii][l], fb[h][j], acc[ii][l][j]);
                }
    };
    // K step h = 0 with the refill of `slot` (stage ksrc of the stream)
    // spread between its MFMAs: a wave that issues all its loads before its
    // MFMAs stalls on the load queue while the matrix pipe idles.
    auto mfma_step_dma = [&](auto first, const int8_t* const (&sp)[LPW], bool do_issue, int slot,
                             int ksrc, bool act) __attribute__((always_inline)) {
        int8_t* st = ring + slot * STAGE;
        if (!act) {
            // no rows of this wave in the tile: only the loads
            if (do_issue)
#pragma unroll
                for (int c = 0; c < LPW; ++c) dma16(sp[c] + (int64_t)ksrc * kKB, st + dst[c]);
            return;
        }
        constexpr int NM = WR * L * 2 * WCP;
        constexpr int PER = NM / LPW > 0 ? NM / LPW : 1;
#pragma unroll
        for (int ii = 0; ii < WR; ++ii)
#pragma unroll
            for (int l = 0; l < L; ++l)
#pragma unroll
                for (int j = 0; j < (2 * WCP); ++j) {
                    if constexpr (decltype(first)::value)
                        acc[ii][l][j] = mfma32(fa[0][ii][l], fb[0][j], v16i{});
                    else
                        acc[ii][l][j] = mfma32(fa[0][ii][l], fb[0][j], acc[ii][l][j]);
                    const int idx = (ii * L + l) * (2 * WCP) + j + 1;
                    if (idx % PER == 0 && idx / PER <= LPW) {
                        __builtin_amdgcn_sched_barrier(0);
                        if (do_issue) dma16(sp[idx / PER - 1] + (int64_t)ksrc * kKB, st + dst[idx / PER - 1]);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
#pragma unroll
        for (int c = NM / PER; c < LPW; ++c)
            if (do_issue) dma16(sp[c] + (int64_t)ksrc * kKB, st + dst[c]);
    };

    // ---- stream prologue: tile 0's rows, metadata and first kS-1 stages
    Info cur = info(0);
    int m = 0;
    fetch_rows(cur, 0);
    wait_vmcnt<0>();
    lds_barrier();
    fetch_row_meta(0);
    // per-lane sources of this wave's loads; from step nk-kS on (when this
    // tile has issued its last stage) they hold the next tile's
    const int8_t* src[LPW];
    make_src(cur, 0, src);
    int slot0 = 0;  // ring slot of the current tile's stage 0
#pragma unroll
    for (int s = 0; s < kS - 1; ++s) issue(s, src, s);

    for (int i = 0; i < tr.ntiles; ++i) {
        const bool has_next = i + 1 < tr.ntiles;
        const int mn = m ^ 1;
        Info nxt = cur;
        if (has_next) nxt = info(i + 1);
        // stage 0 has landed once at most the kS-2 later stages are in flight
        wait_vmcnt<(kS - 2) * LPW>();
        lds_barrier();
        issue((slot0 + kS - 1) % kS, src, kS - 1);
        if (has_next) fetch_rows(nxt, mn);
        // a wave whose rows all lie past the tile's last row (an expert's
        // partial last tile) skips its fragment reads and MFMAs
        const bool act = 32 * WR * wr < cur.nrows;
        if (act) {
            read_frags(slot0, 0);
            read_frags(slot0, 1);
        }
        // One K step: wait for stage ks+1, publish it, refill the slot of
        // stage ks (its fragments are in registers) with stage ks+kS of the
        // stream, and run stage ks while reading stage ks+1's fragments.
        // Phase A (`next` false) refills with this tile's stages; phase B
        // (the last kS steps) with the next tile's first kS-1 stages.
        auto kstep = [&](int ks, auto first, auto next) __attribute__((always_inline)) {
            const int slot = (slot0 + ks) % kS;
            if (ks + 1 < nk) {
                // the stages after ks+1 still in flight are ks+2 .. ks+kS-1
                // of the stream (fewer at the stream's end)
                if (has_next || ks + kS - 1 < nk) wait_vmcnt<(kS - 2) * LPW>();
                else wait_vmcnt<0>();
            }
            lds_barrier();
            const int nslot = (slot + 1) % kS;
            if constexpr (!decltype(next)::value) {
                mfma_step_dma(first, src, true, slot, ks + kS, act);
            } else {
                mfma_step_dma(first, src, has_next && ks + kS - nk <= kS - 2, slot, ks + kS - nk, act);
            }
            if (act) {
                if (ks + 1 < nk) read_frags(nslot, 0);
                mfma_step(1, std::false_type{});
                if (ks + 1 < nk) read_frags(nslot, 1);
            }
        };
        int ks = 0;
        if (nk > kS) {
            kstep(0, std::true_type{}, std::false_type{});
#pragma clang loop unroll(disable)
            for (ks = 1; ks < nk - kS; ++ks) kstep(ks, std::false_type{}, std::false_type{});
        }
        if (has_next) {
            // the next tile's row tokens (fetched at this tile's start) have
            // landed once a stage issued after them has
            if (nk < 2 * kS) {
                wait_vmcnt<0>();
                lds_barrier();
            }
            make_src(nxt, mn, src);
            fetch_row_meta(mn);
        }
        if (ks == 0) {
            kstep(0, std::true_type{}, std::true_type{});
            ks = 1;
        }
#pragma clang loop unroll(disable)
        for (; ks < nk; ++ks) kstep(ks, std::false_type{}, std::true_type{});

        // ---- epilogue (the next tile's first kS-1 stages are in flight):
        // g and u rows out as floats (SiLU and the Z digits follow in
        // swiglu_quant_kernel, at full occupancy).  The zero-point
        // correction is chosen once per tile (zg, zu are uniform), so no
        // per-element test drags its integer multiplies into the common case.
        auto epilogue = [&](auto with_zp) __attribute__((always_inline)) {
            constexpr bool ZP = decltype(with_zp)::value;
            const int e = cur.e, nrows = cur.nrows;
            const float sg = s_sg[e], su = s_su[e];
            const int zg = s_zg[e], zu = s_zu[e];
#pragma unroll
            for (int ii = 0; ii < WR; ++ii) {
                const int r0 = 32 * (wr * WR + ii);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int rq = acc_row(r0, lane, 4 * q);
                    const float4 sx4 = *reinterpret_cast<const float4*>(&s_xs[m][rq]);
                    int4 ds4[L];
                    if constexpr (ZP) {
#pragma unroll
                        for (int l = 0; l < L; ++l) ds4[l] = *reinterpret_cast<const int4*>(&s_xd[m][l][rq]);
                    }
#pragma unroll
                    for (int t4 = 0; t4 < 4; ++t4) {
                        const int v = 4 * q + t4;
                        const float sx = t4 == 0 ? sx4.x : t4 == 1 ? sx4.y : t4 == 2 ? sx4.z : sx4.w;
                        const float fg = __fmul_rn(sx, sg), fu = __fmul_rn(sx, su);
                        const bool live = rq + t4 < nrows;
                        float* grow = gout + (int64_t)(cur.g0 + rq + t4) * I + cur.n0 + 32 * wc * WCP + (lane & 31);
                        float* urow = uout + (grow - gout);
#pragma unroll
                        for (int j = 0; j < WCP; ++j) {
                            int pg[L], pu[L];
#pragma unroll
                            for (int l = 0; l < L; ++l) {
                                pg[l] = acc[ii][l][j][v];
                                pu[l] = acc[ii][l][WCP + j][v];
                            }
                            if constexpr (ZP) {
#pragma unroll
                                for (int l = 0; l < L; ++l) {
                                    const int ds = t4 == 0 ? ds4[l].x : t4 == 1 ? ds4[l].y : t4 == 2 ? ds4[l].z : ds4[l].w;
                                    pg[l] -= zg * ds;
                                    pu[l] -= zu * ds;
                                }
                            }
                            const float g = __fmul_rn(hm_recombine(pg, L), fg);
                            const float u = __fmul_rn(hm_recombine(pu, L), fu);
                            if (live) {
                                grow[32 * j] = g;
                                urow[32 * j] = u;
                            }
                        }
                    }
                }
            }
        };
        if ((s_zg[cur.e] | s_zu[cur.e]) != 0) epilogue(std::true_type{});
        else epilogue(std::false_type{});
        // next tile
        slot0 = (slot0 + nk) % kS;
        m = mn;
        cur = nxt;
    }
}

// ---------------------------------------------------------------------------
// down: tile = BM contiguous grouped rows x BN output columns; wave (wr, wc)
// owns rows [32*WR*wr, +32*WR) and columns [32*WCN*wc, +32*WCN).  After each
// 128-column Z segment (two stages) the exact partials are recombined and
// folded into the float accumulator: acc = fmaf(c, s_segment * scale_down, acc).
// ---------------------------------------------------------------------------
template <int L>
struct DownTile {
    static constexpr int WR = 1;                        // 32-row fragments per wave
    static constexpr int WCN = 2;                       // 32-column fragments per wave
#ifndef HM_DOWN_NWR
#define HM_DOWN_NWR 2
#endif
    static constexpr int NWR = HM_DOWN_NWR, NWC = kWaves / NWR;
    static constexpr int BM = 32 * WR * NWR;            // 64 rows
    static constexpr int BN = 32 * WCN * NWC;           // 256 columns
    static constexpr int NA = L * BM / 32;
    static constexpr int NB = BN / 32;
    static constexpr int NF = NA + NB;
    static constexpr int NL = 2 * NF;
    static constexpr int LPW = (NL + kWaves - 1) / kWaves;
    static constexpr int STAGE = NF * kFragBytes;
    static constexpr int NMETA = (1 + L) * kMaxZSeg * (BM / HM_WAVE);  // metadata DMAs per tile
};

template <int L>
__global__ __launch_bounds__(kThreads) void down_mfma_kernel(
    const int8_t* __restrict__ zdig, const float* __restrict__ zscale,
    const int32_t* __restrict__ zdsum, int R, int H, int I, int experts,
    const int8_t* __restrict__ packed, const float* __restrict__ scale,
    const int32_t* __restrict__ zp, const int32_t* __restrict__ counts,
    const int32_t* __restrict__ offsets, float* __restrict__ y) {
    using T = DownTile<L>;
    constexpr int kSD = down_stages<L>();
    constexpr int BM = T::BM, BN = T::BN, NA = T::NA, NL = T::NL, LPW = T::LPW, WR = T::WR,
                  WCN = T::WCN, NWC = T::NWC, STAGE = T::STAGE;
    constexpr int RC = BM / HM_WAVE;  // 64-row chunks of a tile
    __shared__ __attribute__((aligned(1024))) int8_t ring[kSD * STAGE];
    __shared__ int32_t s_prefix[kMaxExperts + 1];
    __shared__ int32_t s_off[kMaxExperts], s_cnt[kMaxExperts];
    __shared__ float s_sd[kMaxExperts];
    __shared__ int32_t s_zd[kMaxExperts];
    __shared__ __attribute__((aligned(16))) float s_zs[2][kMaxZSeg][BM];       // Z segment scales
    __shared__ __attribute__((aligned(16))) int32_t s_zds[2][L][kMaxZSeg][BM]; // Z digit sums

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = wave / NWC, wc = wave % NWC;
    const int E = (int)experts;
    for (int e = tid; e < E; e += kThreads) {
        s_cnt[e] = counts[e];
        s_off[e] = offsets[e];
        s_sd[e] = scale[3 * e + 2];
        s_zd[e] = zp[3 * e + 2];
    }
    __syncthreads();
    if (wave == 0) tile_prefix(s_cnt, E, BM, s_prefix);
    __syncthreads();
    const int nbn = H / BN;
    const TileRange tr = tile_range(s_prefix[E] * nbn);
    if (tr.ntiles == 0) return;
    const int nk = (int)(I / kKB);
    const int nbz = (int)(I / kZBlock);

    struct Info {
        int e, nrows, g0, n0;
    };
    auto info = [&](int i) __attribute__((always_inline)) {
        const int j = tr.jbeg + i * tr.step;
        const int gm = j / nbn;
        Info t;
        t.e = locate_expert(s_prefix, E, gm);
        const int mt = gm - s_prefix[t.e];
        t.g0 = s_off[t.e] + mt * BM;
        t.nrows = min(BM, s_cnt[t.e] - mt * BM);
        t.n0 = (j % nbn) * BN;
        return t;
    };
    // Z segment scales and digit sums of the tile rows (rows past nrows read
    // the last row); units spread over the waves
    auto fetch_meta = [&](const Info& t, int m) __attribute__((always_inline)) {
        for (int u = wave; u < (1 + L) * nbz * RC; u += kWaves) {
            const int kind = u / (nbz * RC), rem = u % (nbz * RC);
            const int b = rem / RC, ch = rem % RC;
            const int r = HM_WAVE * ch + lane;
            const int64_t g = t.g0 + min(r, t.nrows - 1);
            if (kind == 0) dma4(zscale + g * nbz + b, &s_zs[m][b][HM_WAVE * ch]);
            else dma4(zdsum + ((int64_t)(kind - 1) * R + g) * nbz + b, &s_zds[m][kind - 1][b][HM_WAVE * ch]);
        }
    };
    int dst[LPW];
#pragma unroll
    for (int c = 0; c < LPW; ++c) {
        const int u = (wave + kWaves * c) % NL;
        dst[c] = (u >> 1) * kFragBytes + 1024 * (u & 1);
    }
    auto make_src = [&](const Info& t, const int8_t* (&src)[LPW]) {
        const int8_t* dbase = packed + (int64_t)t.e * 3 * H * I + 2 * H * I;
        const int ch = frag_load_chunk(lane);
#pragma unroll
        for (int c = 0; c < LPW; ++c) {
            const int u = (wave + kWaves * c) % NL;
            const int f = u >> 1, row = frag_load_row(lane, u & 1);
            if (f < NA) {
                const int l = f / (BM / 32), i = f % (BM / 32);
                const int r = 32 * i + row;
                src[c] = zdig + ((int64_t)l * R + t.g0 + min(r, t.nrows - 1)) * I + 16 * ch;
            } else {
                src[c] = dbase + (t.n0 + 32 * (f - NA) + row) * I + 16 * ch;
            }
        }
    };
    auto issue = [&](int slot, const int8_t* const (&src)[LPW], int ks) {
        int8_t* st = ring + slot * STAGE;
#pragma unroll
        for (int c = 0; c < LPW; ++c) dma16(src[c] + (int64_t)ks * kKB, st + dst[c]);
    };

    int rd[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) rd[h] = frag_read_offset(lane, h);
    v4i fa[2][WR][L], fb[2][WCN];
    auto read_frags = [&](int slot, int h) __attribute__((always_inline)) {
        const int8_t* st = ring + slot * STAGE;
#pragma unroll
        for (int ii = 0; ii < WR; ++ii)
#pragma unroll
            for (int l = 0; l < L; ++l)
                fa[h][ii][l] = lds16(st + (l * (BM / 32) + wr * WR + ii) * kFragBytes + rd[h]);
#pragma unroll
        for (int j = 0; j < WCN; ++j) fb[h][j] = lds16(st + (NA + wc * WCN + j) * kFragBytes + rd[h]);
    };
    v16i acc[WR][L][WCN];
    float facc[WR][WCN][16];
    // `first`: the first K step of a Z segment starts the partials from zero
    auto mfma_step = [&](int h, auto first) __attribute__((always_inline)) {
#pragma unroll
        for (int ii = 0; ii < WR; ++ii)
#pragma unroll
            for (int l = 0; l < L; ++l)
#pragma unroll
                for (int j = 0; j < WCN; ++j) {
                    if constexpr (decltype(first)::value)
                        acc[ii][l][j] = mfma32(fa[h][ii][l], fb[h][j], v16i{});
                    else
                        acc[ii][l][j] = mfma32(fa[h][ii][l], fb[h][j], acc[ii][l][j]);
                }
    };
    // K step h = 0 with the refill of `slot` (stage ksrc of the stream)
    // spread between its MFMAs: a wave that issues all its loads before its
    // MFMAs stalls on the load queue while the matrix pipe idles.
    auto mfma_step_dma = [&](auto first, const int8_t* const (&sp)[LPW], bool do_issue, int slot,
                             int ksrc, bool act) __attribute__((always_inline)) {
        int8_t* st = ring + slot * STAGE;
        if (!act) {
            // no rows of this wave in the tile: only the loads
            if (do_issue)
#pragma unroll
                for (int c = 0; c < LPW; ++c) dma16(sp[c] + (int64_t)ksrc * kKB, st + dst[c]);
            return;
        }
        constexpr int NM = WR * L * WCN;
        constexpr int PER = NM / LPW > 0 ? NM / LPW : 1;
#pragma unroll
        for (int ii = 0; ii < WR; ++ii)
#pragma unroll
            for (int l = 0; l < L; ++l)
#pragma unroll
                for (int j = 0; j < WCN; ++j) {
                    if constexpr (decltype(first)::value)
                        acc[ii][l][j] = mfma32(fa[0][ii][l], fb[0][j], v16i{});
                    else
                        acc[ii][l][j] = mfma32(fa[0][ii][l], fb[0][j], acc[ii][l][j]);
                    const int idx = (ii * L + l) * WCN + j + 1;
                    if (idx % PER == 0 && idx / PER <= LPW) {
                        __builtin_amdgcn_sched_barrier(0);
                        if (do_issue) dma16(sp[idx / PER - 1] + (int64_t)ksrc * kKB, st + dst[idx / PER - 1]);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
#pragma unroll
        for (int c = NM / PER; c < LPW; ++c)
            if (do_issue) dma16(sp[c] + (int64_t)ksrc * kKB, st + dst[c]);
    };

    Info cur = info(0);
    int m = 0;
    fetch_meta(cur, 0);
    const int8_t* src[LPW];  // this tile's sources, the next tile's from step nk-kSD
    make_src(cur, src);
    int slot0 = 0;
#pragma unroll
    for (int s = 0; s < kSD - 1; ++s) issue(s, src, s);

    for (int i = 0; i < tr.ntiles; ++i) {
        const bool has_next = i + 1 < tr.ntiles;
        const int mn = m ^ 1;
        Info nxt = cur;
        if (has_next) nxt = info(i + 1);
        wait_vmcnt<(kSD - 2) * LPW>();
        lds_barrier();
        issue((slot0 + kSD - 1) % kSD, src, kSD - 1);
        if (has_next) fetch_meta(nxt, mn);
        // a wave whose rows all lie past the tile's last row (an expert's
        // partial last tile) skips its fragment reads and MFMAs
        const bool act = 32 * WR * wr < cur.nrows;
        if (act) {
            read_frags(slot0, 0);
            read_frags(slot0, 1);
        }
        const float sd = s_sd[cur.e];
        const int zd = s_zd[cur.e];
#pragma unroll
        for (int ii = 0; ii < WR; ++ii)
#pragma unroll
            for (int j = 0; j < WCN; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) facc[ii][j][v] = 0.0f;
        auto dstep = [&](int ks, auto first, auto next) __attribute__((always_inline)) {
            const int slot = (slot0 + ks) % kSD;
            if (ks + 1 < nk) {
                if (has_next || ks + kSD - 1 < nk) wait_vmcnt<(kSD - 2) * LPW>();
                else wait_vmcnt<0>();
            }
            lds_barrier();
            const int nslot = (slot + 1) % kSD;
            if constexpr (!decltype(next)::value) {
                mfma_step_dma(first, src, true, slot, ks + kSD, act);
            } else {
                mfma_step_dma(first, src, has_next && ks + kSD - nk <= kSD - 2, slot, ks + kSD - nk, act);
            }
            if (act) {
                if (ks + 1 < nk) read_frags(nslot, 0);
                mfma_step(1, std::false_type{});
                if (ks + 1 < nk) read_frags(nslot, 1);
            }
        };
        // end of Z segment zb: exact partials -> float.  Within one 128-wide
        // segment |P_l| <= 2^22 (with a zero-point correction), so two
        // limbs combine exactly in int32 and convert with the single
        // rounding of fmaf((float)P_1, 256, (float)P_0).
        // The zero-point correction is chosen once per tile (zd is uniform):
        // a per-element test would let the compiler hoist its integer
        // multiplies out of the branch into every fold.
        auto fold = [&](int zb, auto with_zp) __attribute__((always_inline)) {
            constexpr bool ZP = decltype(with_zp)::value;
#pragma unroll
            for (int ii = 0; ii < WR; ++ii)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int rq = acc_row(32 * (wr * WR + ii), lane, 4 * q);
                    const float4 zs4 = *reinterpret_cast<const float4*>(&s_zs[m][zb][rq]);
                    int4 dz4[L];
                    if constexpr (ZP) {
#pragma unroll
                        for (int l = 0; l < L; ++l) dz4[l] = *reinterpret_cast<const int4*>(&s_zds[m][l][zb][rq]);
                    }
#pragma unroll
                    for (int t4 = 0; t4 < 4; ++t4) {
                        const int v = 4 * q + t4;
                        const float zs = t4 == 0 ? zs4.x : t4 == 1 ? zs4.y : t4 == 2 ? zs4.z : zs4.w;
                        const float alpha = __fmul_rn(zs, sd);
                        int dzc[L];
                        if constexpr (ZP) {
#pragma unroll
                            for (int l = 0; l < L; ++l)
                                dzc[l] = zd * (t4 == 0 ? dz4[l].x : t4 == 1 ? dz4[l].y : t4 == 2 ? dz4[l].z : dz4[l].w);
                        }
#pragma unroll
                        for (int j = 0; j < WCN; ++j) {
                            int p[L];
#pragma unroll
                            for (int l = 0; l < L; ++l) p[l] = acc[ii][l][j][v];
                            if constexpr (ZP) {
#pragma unroll
                                for (int l = 0; l < L; ++l) p[l] -= dzc[l];
                            }
                            float c;
                            if constexpr (L == 1) c = (float)p[0];
                            else if constexpr (L == 2) c = (float)(p[1] * 256 + p[0]);
                            else c = hm_recombine(p, L);
                            facc[ii][j][v] = __builtin_fmaf(c, alpha, facc[ii][j][v]);
                        }
                    }
                }
        };
        auto fold_seg = [&](int zb) __attribute__((always_inline)) {
            if (!act) return;
            if (zd != 0) fold(zb, std::true_type{});
            else fold(zb, std::false_type{});
        };
        // A Z segment is two stages (nk is even); phase B (the last kSD
        // steps) may start inside one when kSD is odd.
        int ks = 0;
#pragma clang loop unroll(disable)
        for (; ks + 1 < nk - kSD; ks += 2) {
            dstep(ks, std::true_type{}, std::false_type{});
            dstep(ks + 1, std::false_type{}, std::false_type{});
            fold_seg(ks >> 1);
        }
        if (ks < nk - kSD) {
            dstep(ks, std::true_type{}, std::false_type{});
            if (has_next) make_src(nxt, src);
            dstep(ks + 1, std::false_type{}, std::true_type{});
            fold_seg(ks >> 1);
            ks += 2;
        } else if (has_next) {
            make_src(nxt, src);
        }
#pragma clang loop unroll(disable)
        for (; ks < nk; ks += 2) {
            dstep(ks, std::true_type{}, std::true_type{});
            dstep(ks + 1, std::false_type{}, std::true_type{});
            fold_seg(ks >> 1);
        }
        // ---- epilogue: float rows out (the next tile's stages are in flight)
#pragma unroll
        for (int ii = 0; ii < WR; ++ii)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int r = acc_row(32 * (wr * WR + ii), lane, v);
            if (r < cur.nrows) {
                float* yr = y + (cur.g0 + r) * H + cur.n0 + 32 * wc * WCN + (lane & 31);
#pragma unroll
                for (int j = 0; j < WCN; ++j) yr[32 * j] = facc[ii][j][v];
            }
        }
        slot0 = (slot0 + nk) % kSD;
        m = mn;
        cur = nxt;
    }
}

// ---------------------------------------------------------------------------
// z = silu(g) * u and its fixed-point digits: one half-wave per 128-column
// segment of a grouped row (lane: columns 4*(lane%32) .. +3 of segment
// 2*wave_id + lane/32).  The segment max gives the step: inv = range /
// max|z|, digits of rint(z * inv); the segment scale max|z| / range and the
// digit sums go out beside them.  The same arithmetic as
// zquant_generic_kernel over the z of gateup_generic_kernel.
// ---------------------------------------------------------------------------
constexpr int kSqThreads = 256;

// Max / integer sum over each 32-lane half of the wave (both halves at once).
__device__ __forceinline__ float half_wave_max(float v) {
    const float r = hm_row16_max(v);
    const int lane = threadIdx.x & (HM_WAVE - 1);
    const int b = __builtin_bit_cast(int, r);
    const float a0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
    const float a1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
    const float a2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
    const float a3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
    return lane < 32 ? fmaxf(a0, a1) : fmaxf(a2, a3);
}
__device__ __forceinline__ int half_wave_sum(int v) {
    const int r = hm_row16_sum(v);
    const int lane = threadIdx.x & (HM_WAVE - 1);
    const int s0 = __builtin_amdgcn_readlane(r, 0) + __builtin_amdgcn_readlane(r, 16);
    const int s1 = __builtin_amdgcn_readlane(r, 32) + __builtin_amdgcn_readlane(r, 48);
    return lane < 32 ? s0 : s1;
}

template <int L>
__global__ __launch_bounds__(kSqThreads) void swiglu_quant_kernel(
    const float* __restrict__ gin, const float* __restrict__ uin, int R, int I,
    int8_t* __restrict__ zdig, float* __restrict__ zscale, int32_t* __restrict__ zdsum) {
    __shared__ unsigned long long s_exp2[32];
    hm_load_exp2_table(s_exp2);
    __syncthreads();
    const int lane = threadIdx.x & (HM_WAVE - 1);
    const int nbz = I / kZBlock;
    const int pair = blockIdx.x * (kSqThreads / HM_WAVE) + (int)(threadIdx.x / HM_WAVE);
    if (2 * pair >= R * nbz) return;
    // a wave's two segments; an odd total leaves the last wave's upper half
    // on a repeat of its lower segment (computed, not stored)
    const int seg_raw = 2 * pair + (lane >> 5);
    const bool store = seg_raw < R * nbz;
    const int seg = store ? seg_raw : 2 * pair;
    const int row = seg / nbz, b = seg % nbz;
    const int64_t off = (int64_t)row * I + b * kZBlock + 4 * (lane & 31);
    const float4 g = *reinterpret_cast<const float4*>(gin + off);
    const float4 u = *reinterpret_cast<const float4*>(uin + off);
    float sv[4];
    const float gv[4] = {g.x, g.y, g.z, g.w};
    if (__all(fabsf(g.x) < 88.0f && fabsf(g.y) < 88.0f && fabsf(g.z) < 88.0f && fabsf(g.w) < 88.0f)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[i] = hm_silu_small_t(gv[i], s_exp2);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[i] = hm_silu_t(gv[i], s_exp2);
    }
    const float z[4] = {__fmul_rn(sv[0], u.x), __fmul_rn(sv[1], u.y), __fmul_rn(sv[2], u.z),
                        __fmul_rn(sv[3], u.w)};
    const float amax = half_wave_max(fmaxf(fmaxf(fabsf(z[0]), fabsf(z[1])), fmaxf(fabsf(z[2]), fabsf(z[3]))));
    const float range = (float)hm_limb_range(L);
    const float inv = amax > 0.0f ? __fdiv_rn(range, amax) : 0.0f;
    int d[4][L];
#pragma unroll
    for (int i = 0; i < 4; ++i) hm_digits<L>(hm_fixed_point(z[i], inv, range), d[i]);
#pragma unroll
    for (int l = 0; l < L; ++l) {
        const uint32_t word = (uint32_t)(d[0][l] & 255) | ((uint32_t)(d[1][l] & 255) << 8) |
                              ((uint32_t)(d[2][l] & 255) << 16) | ((uint32_t)(d[3][l] & 255) << 24);
        if (store) *reinterpret_cast<uint32_t*>(zdig + (int64_t)l * R * I + off) = word;
        const int sum = half_wave_sum(d[0][l] + d[1][l] + d[2][l] + d[3][l]);
        if (store && (lane & 31) == 0) zdsum[((int64_t)l * R + row) * nbz + b] = sum;
    }
    if (store && (lane & 31) == 0)
        zscale[(int64_t)row * nbz + b] = amax > 0.0f ? __fdiv_rn(amax, range) : 0.0f;
}

int persistent_grid() {
    static int cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (cached[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        cached[dev] = cus;
    }
    const int g = cached[dev] / kXcds * kXcds;
    return g < kXcds ? kXcds : g;
}

template <int L>
int launch_gateup(const hm_layer* layer, const int8_t* xdig, const float* xscale,
                  const int32_t* xdsum, int64_t tokens, const int32_t* counts,
                  const int32_t* offsets, const int32_t* perm_tokens, int64_t R, float* gu,
                  int8_t* zdig, float* zscale, int32_t* zdsum, hipStream_t stream) {
    const int64_t I = layer->intermediate;
    if (tokens > INT_MAX || R > INT_MAX || R * (I / kZBlock) > INT_MAX) return HM_ERR_OVERFLOW;
    float* gout = gu;
    float* uout = gu + R * I;
    HM_STAGE_LAUNCH(true, false, gateup_mfma_kernel<L>, dim3((unsigned)persistent_grid()),
                    dim3(kThreads), 0, stream, xdig, xscale, xdsum, (int)tokens,
                    (int)layer->hidden, (int)I, (int)layer->experts,
                    static_cast<const int8_t*>(layer->packed), layer->scale, layer->zero_point,
                    counts, offsets, perm_tokens, (int)R, gout, uout);
    HM_LAUNCHED();
    const int64_t pairs = (R * (I / kZBlock) + 1) / 2;
    const int64_t per_block = kSqThreads / HM_WAVE;
    HM_STAGE_LAUNCH(false, true, swiglu_quant_kernel<L>,
                    dim3((unsigned)((pairs + per_block - 1) / per_block)), dim3(kSqThreads), 0,
                    stream, gout, uout, (int)R, (int)I, zdig, zscale, zdsum);
    HM_LAUNCHED();
    return HM_OK;
}

template <int L>
int launch_down(const hm_layer* layer, const int32_t* counts, const int32_t* offsets, int64_t R,
                const int8_t* zdig, const float* zscale, const int32_t* zdsum, float* y,
                hipStream_t stream) {
    if (R > INT_MAX) return HM_ERR_OVERFLOW;
    hipLaunchKernelGGL(down_mfma_kernel<L>, dim3((unsigned)persistent_grid()), dim3(kThreads), 0,
                       stream, zdig, zscale, zdsum, (int)R, (int)layer->hidden,
                       (int)layer->intermediate, (int)layer->experts,
                       static_cast<const int8_t*>(layer->packed), layer->scale, layer->zero_point,
                       counts, offsets, y);
    HM_LAUNCHED();
    return HM_OK;
}

}  // namespace

// Shape preconditions of the MFMA kernels.  gate/up: K = H in 64-byte
// stages, at least kS of them; I in 128-column blocks.  down: K = I in
// 64-byte stages (at least kS), 128-wide Z segments (at most kMaxZSeg held
// per row), H in tiles of the down tile width.  Both keep the expert
// tables in LDS (E <= kMaxExperts).
bool hm_mfma_gateup_ok(int64_t H, int64_t I, int64_t E, int32_t limbs) {
    // |P_l| <= H * 128 * 255 < 2^31 keeps every limb partial exact: H <= 65536
    return limbs >= 1 && limbs <= 3 && E >= 1 && E <= kMaxExperts && H <= 65536 &&
           I <= (1 << 20) && H % kKB == 0 &&
           H / kKB >= kS && I % kGateUpN == 0 && I >= kGateUpN;
}

bool hm_mfma_down_ok(int64_t H, int64_t I, int64_t E, int32_t limbs) {
    if (limbs < 1 || limbs > 3 || E < 1 || E > kMaxExperts || H > (1 << 20) || I > (1 << 20))
        return false;
    const int64_t bn = limbs == 1 ? DownTile<1>::BN : limbs == 2 ? DownTile<2>::BN : DownTile<3>::BN;
    const int64_t st = limbs == 1 ? down_stages<1>() : limbs == 2 ? down_stages<2>() : down_stages<3>();
    return H % bn == 0 && H >= bn && I % kZBlock == 0 && I / kKB >= st && I / kZBlock <= kMaxZSeg;
}

// gu: scratch for the exact g and u rows, 2 x R x I floats.
int hm_launch_gateup_i8_mfma(const hm_layer* layer, int32_t limbs, const int8_t* xdig,
                             const float* xscale, const int32_t* xdsum, int64_t tokens,
                             const int32_t* counts, const int32_t* offsets,
                             const int32_t* perm_tokens, int64_t R, float* gu, int8_t* zdig,
                             float* zscale, int32_t* zdsum, hipStream_t stream) {
    switch (limbs) {
    case 1: return launch_gateup<1>(layer, xdig, xscale, xdsum, tokens, counts, offsets, perm_tokens, R, gu, zdig, zscale, zdsum, stream);
    case 2: return launch_gateup<2>(layer, xdig, xscale, xdsum, tokens, counts, offsets, perm_tokens, R, gu, zdig, zscale, zdsum, stream);
    case 3: return launch_gateup<3>(layer, xdig, xscale, xdsum, tokens, counts, offsets, perm_tokens, R, gu, zdig, zscale, zdsum, stream);
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
