// hm_gemm_mfma.hip -- grouped INT8-MFMA expert GEMMs for gfx950.
//
// One kernel template serves both projections of the expert MLP:
//   gate/up  A = the token rows' X digit planes (gathered by perm_tokens),
//            B = the gate and up tiles; epilogue z = silu(g) * u -> floats.
//   down     A = the grouped rows' Z digit planes (contiguous),
//            B = the down tiles; epilogue y -> floats.
// The activation operand is L fixed-point digit planes with one scale per
// row (hm_device.h); every plane meets the same weight fragment in one
// v_mfma_i32_32x32x32_i8, so each plane's int32 partial over the whole row
// is exact, and the epilogue recombines them (hm_recombine) exactly as the
// generic kernels and the CPU restatement do.
//
// Operand layout of v_mfma_i32_32x32x32_i8: lane l supplies 16 bytes of row
// l % 32 of A and of column l % 32 of B, K bytes 16 (l / 32) .. +15 of the
// 32-wide step; its 16 int32 results are column l % 32, rows
// 8 (v / 4) + 4 (l / 32) + v % 4 (v = 0..15).
//
// Workgroup: 4 wave64s (one per SIMD, up to 512 registers each: the
// accumulators take the AGPRs), persistent, one per CU.  A tile is BM
// grouped rows of one expert x the workgroup's columns; every wave holds all
// BM rows and its own two 32-column fragments:
//   gate/up  wave w: gate and up columns 32 w .. +31 of a 128-column block
//            of z (the same n, so z = silu(g) * u is lane-local)
//   down     wave w: output columns 64 w .. +63 of a 256-column block
//
// Data movement, per stage of K = 128 bytes (four MFMA K steps):
//   A  global -> LDS by 16-byte global_load_lds (inline asm), 128-byte row
//      chunks (whole cache lines), into a ring of kSA stages.  Each row's
//      eight 16-byte chunks are stored rotated by (row >> 1) & 7, so the
//      readers' ds_read_b128 over any 16 lanes hit 16 distinct bank groups.
//   B  global -> VGPRs: the weights are stored as 1 KB tiles in operand
//      order (hm_tile_offset), so one 16-byte-per-lane load is one B
//      fragment, read as one contiguous kilobyte; a ring of DB stages of
//      registers.
// Every wave issues its share of the loads of later stages between the
// MFMAs of the current one (a wave that issues its loads in a clump stalls
// the matrix pipe behind them).  Stages form one stream per workgroup across
// its tiles, so the next tile's first stages load while the current tile
// finishes.  The LDS DMA is invisible to the compiler: the kernel waits for
// it with explicit vmcnt counts (every vector memory instruction between the
// awaited load and the wait is counted; stores and metadata loads only add
// to the count, which keeps the wait conservative).
//
// Tile order: tiles are numbered m-tile major, column block minor, and split
// into 8 contiguous ranges, one per XCD (workgroup i runs on XCD i % 8), so
// the column blocks of an m-tile (sharing A rows) and the m-tiles of one
// expert (sharing B tiles) meet in one XCD's L2.  In an expert's partial
// last tile, the 32-row fragments past its last row skip their reads and
// MFMAs.
#include "hm_device.h"
#include "hm_lds_dma.h"

#include <limits.h>

#include <type_traits>

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kKS = 128;            // K bytes per stage
constexpr int kKT = kKS / 32;       // MFMA K steps per stage
constexpr int kSA = 4;              // A ring stages (LDS)
constexpr int kXcds = 8;
constexpr int kMaxExperts = 256;    // expert tables live in LDS

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

enum Role { kGateUp = 0, kDown = 1 };

template <int ROLE, int L, int DB>
struct Tile {
    static constexpr int RF = L <= 2 ? 4 : 2;            // 32-row fragments per tile
    static constexpr int BM = 32 * RF;                   // tile rows
    static constexpr int NCF = 2;                        // 32-column fragments per wave
    static constexpr int BN = ROLE == kGateUp ? 32 * kWaves : 32 * NCF * kWaves;  // output columns
    static constexpr int ASTAGE = L * BM * kKS;          // A bytes per stage
    static constexpr int ALOADS = ASTAGE / 1024;         // wave-wide A loads per stage
    static constexpr int APW = ALOADS / kWaves;          // ... per wave
    static constexpr int BPW = NCF * kKT;                // B loads per wave per stage
    static constexpr int NV = APW + BPW;                 // loads per wave per stage
    static constexpr int NG = kKT * RF;                  // (K step, row fragment) groups per stage
    static_assert(ALOADS % kWaves == 0 && APW <= BPW && DB >= 2 && DB <= kSA && kKT % 2 == 0,
                  "tile shape");
    // A stage's load items: its B loads first (the compiler's waits for the
    // B registers do not see the DMAs, so a DMA issued after a B load is
    // only waited for where that B load is), then its A DMAs; item j is
    // issued before group item_group(j) of the stage.
    static constexpr bool item_is_a(int j) { return j >= BPW; }
    static constexpr int item_a(int j) { return j - BPW; }
    static constexpr int item_b(int j) { return j; }
    static constexpr int item_group(int j) { return j * NG / NV; }
    // the wait of a stage comes before its last K step's groups
    static constexpr int kWaitGroup = (kKT - 1) * RF;
    static constexpr int items_before(int g) {
        int n = 0;
        for (int j = 0; j < NV; ++j) n += item_group(j) < g ? 1 : 0;
        return n;
    }
    // loads after the last DMA of a stage, within that stage
    static constexpr int after_last_a = 0;
    // At the wait of stage g for A(g+1), whose DMAs stage g+2-kSA issued:
    // the loads issued since that stage's last DMA.
    static constexpr int wait_count = after_last_a + (kSA - 3) * NV + items_before(kWaitGroup);
    static_assert(wait_count <= 63, "vmcnt");
};

// One wave-wide 16-byte buffer -> LDS load: lane l's 16 bytes from
// rsrc + voff + soff land at lds_base + 16 l (M0 holds the wave-uniform LDS
// base; the statement sets it itself, as dma16 does).  Loads past the
// buffer's size return zeros instead of faulting.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff, uint32_t soff,
                                          void* lds_base) {
    const unsigned m0 = (unsigned)(uintptr_t)(lds_ptr_t)lds_base;
    asm volatile("s_mov_b32 m0, %3\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
                 ::"v"(voff), "s"(rsrc), "s"(soff), "s"(m0) : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// The lane index, recomputed where it is used: derived per-lane constants
// are then formed at their (once-per-tile) use instead of being hoisted out
// of the tile loop, where they would occupy registers the accumulator
// pipeline needs.
__device__ __forceinline__ int fresh_lane() {
    int v = (int)(threadIdx.x & 63);
    asm volatile("" : "+v"(v));
    return v;
}

__device__ __forceinline__ v16i mfma32(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// Position of 16-byte chunk c of ring row r (rotated by the row); its own
// inverse in c.
__device__ __forceinline__ int a_chunk_pos(int r, int c) { return c ^ ((r >> 1) & 7); }

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
// (experts with no tiles share their successor's start and are skipped).
// Every lane of the wave must be active.
__device__ __forceinline__ int locate_expert(const int32_t* prefix, int E, int gm) {
    const int lane = threadIdx.x & (HM_WAVE - 1);
    int n = 0;
    for (int c0 = 0; c0 < E; c0 += HM_WAVE) {
        const int e = c0 + lane;
        n += __popcll(__ballot(e < E && prefix[e] <= gm));
    }
    return __builtin_amdgcn_readfirstlane(n - 1);
}

// The workgroup's tiles: jbeg, jbeg + step, ... < jend of its XCD's range.
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

struct TileInfo {
    int e, nrows, g0, n0;
};

// ---------------------------------------------------------------------------
// The grouped limb GEMM.
//   gate/up: K = H, N = I (z columns), out = zf [R x I]
//   down:    K = I, N = H, out = y [R x H]
// A rows: gate/up adig [L][tokens][K] gathered by perm_tokens; down adig
// [L][R][K] by grouped row.  ascale/adsum: the A rows' fixed-point scales
// [arows] and digit sums [L][arows] (for non-zero zero points).
// ---------------------------------------------------------------------------
template <int ROLE, int L, int DB>
__global__ __launch_bounds__(kThreads) void limb_gemm_kernel(
    const int8_t* __restrict__ adig, const float* __restrict__ ascale,
    const int32_t* __restrict__ adsum, int arows, int K, int N, int H, int I, int experts,
    const int8_t* __restrict__ packed, const float* __restrict__ scale,
    const int32_t* __restrict__ zp, const int32_t* __restrict__ counts,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ perm_tokens,
    float* __restrict__ out) {
    using T = Tile<ROLE, L, DB>;
    constexpr int RF = T::RF, BM = T::BM, BN = T::BN, NCF = T::NCF, APW = T::APW,
                  BPW = T::BPW, NV = T::NV, ASTAGE = T::ASTAGE;
    constexpr bool GU = ROLE == kGateUp;
    constexpr int MW = BM / HM_WAVE;  // 64-row metadata chunks of a tile
    __shared__ __attribute__((aligned(1024))) int8_t ring[kSA * ASTAGE];
    __shared__ int32_t s_prefix[kMaxExperts + 1];
    __shared__ int32_t s_off[kMaxExperts], s_cnt[kMaxExperts];
    __shared__ float s_sa[kMaxExperts], s_sb[kMaxExperts];     // gate (or down), up scale
    __shared__ int32_t s_za[kMaxExperts], s_zb[kMaxExperts];   // and zero points
    __shared__ __attribute__((aligned(16))) int32_t s_rt[2][BM];     // gate/up: token of each row
    __shared__ __attribute__((aligned(16))) float s_as[2][BM];       // A row scale
    __shared__ __attribute__((aligned(16))) int32_t s_ad[2][L][BM];  // A row digit sums
    __shared__ unsigned long long s_exp2[32];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int E = experts;
    for (int e = tid; e < E; e += kThreads) {
        s_cnt[e] = counts[e];
        s_off[e] = offsets[e];
        s_sa[e] = scale[3 * e + (GU ? 0 : 2)];
        s_sb[e] = scale[3 * e + 1];
        s_za[e] = zp[3 * e + (GU ? 0 : 2)];
        s_zb[e] = zp[3 * e + 1];
    }
    if (GU) hm_load_exp2_table(s_exp2);
    __syncthreads();
    if (wave == 0) tile_prefix(s_cnt, E, BM, s_prefix);
    __syncthreads();
    const int nbn = N / BN;
    const TileRange tr = tile_range(s_prefix[E] * nbn);
    if (tr.ntiles == 0) return;
    const int nk = K / kKS;                  // stages per tile (a multiple of DB)
    const int G = tr.ntiles * nk;            // stages of the workgroup's stream
    const int64_t K32 = hm_pad32(K);

    auto info = [&](int i) __attribute__((always_inline)) {
        const int j = tr.jbeg + i * tr.step;
        const int gm = j / nbn;
        TileInfo t;
        t.e = locate_expert(s_prefix, E, gm);
        const int mt = gm - s_prefix[t.e];
        t.g0 = s_off[t.e] + mt * BM;
        t.nrows = min(BM, s_cnt[t.e] - mt * BM);
        t.n0 = (j % nbn) * BN;
        return t;
    };
    // gate/up: the token ids of a tile's rows (rows past nrows repeat the
    // last row) into s_rt[m]
    auto fetch_tokens = [&](const TileInfo& t, int m) __attribute__((always_inline)) {
        if constexpr (GU) {
            if (wave < MW) {
                const int r = HM_WAVE * wave + fresh_lane();
                dma4(perm_tokens + t.g0 + min(r, t.nrows - 1), &s_rt[m][HM_WAVE * wave]);
            }
        }
    };
    // the A rows' scales and digit sums into s_as[m], s_ad[m] (gate/up: reads
    // s_rt[m], which must be visible)
    auto fetch_meta = [&](const TileInfo& t, int m) __attribute__((always_inline)) {
        if (wave < MW) {
            const int r = HM_WAVE * wave + fresh_lane();
            const int src = GU ? s_rt[m][r] : t.g0 + min(r, t.nrows - 1);
            dma4(ascale + src, &s_as[m][HM_WAVE * wave]);
#pragma unroll
            for (int l = 0; l < L; ++l)
                dma4(adsum + (int64_t)l * arows + src, &s_ad[m][l][HM_WAVE * wave]);
        }
    };

    // ---- load sources of a tile (buffer resources: wave-uniform bases,
    // 32-bit per-lane offsets)
    // A: load unit u = wave + kWaves i covers ring rows 8u .. 8u+7 (limb-major
    // [L][BM], 128 bytes a row); lane: row 8u + lane/8, ring position lane%8,
    // which holds chunk a_chunk_pos(row, lane%8) of the row.
    const __amdgpu_buffer_rsrc_t arsrc = buffer_rsrc(adig, (uint32_t)((int64_t)L * arows * K));
    uint32_t aoff[APW];
    auto make_asrc = [&](const TileInfo& t, int m) __attribute__((always_inline)) {
        const int ln = fresh_lane();
#pragma unroll
        for (int i = 0; i < APW; ++i) {
            const int q = 8 * (wave + kWaves * i) + (ln >> 3);
            const int l = q / BM, r = q % BM;
            const int c = a_chunk_pos(r, ln & 7);
            const int row = GU ? s_rt[m][r] : t.g0 + min(r, t.nrows - 1);
            aoff[i] = (uint32_t)(((int64_t)l * arows + row) * K + 16 * c);
        }
    };
    // B: the tile's expert as one buffer; fragment f's K tiles are
    // contiguous from boff[f] (uniform) + 16 lane
    __amdgpu_buffer_rsrc_t brsrc;
    int boff[NCF];
    const uint32_t blane = 16u * (uint32_t)lane;
    auto make_bsrc = [&](const TileInfo& t) __attribute__((always_inline)) {
        brsrc = buffer_rsrc(packed + hm_proj_offset(t.e, 0, H, I), (uint32_t)(3 * hm_proj_bytes(H, I)));
#pragma unroll
        for (int f = 0; f < NCF; ++f) {
            const int p = GU ? f : 2;
            const int cb = GU ? t.n0 / 32 + wave : t.n0 / 32 + NCF * wave + f;
            boff[f] = (int)(p * hm_proj_bytes(H, I) + (int64_t)cb * (K32 / 32) * 1024);
        }
    };
    auto issue_a = [&](int i, int stage, int ks) __attribute__((always_inline)) {
        dma16_buf(arsrc, aoff[i], (uint32_t)(ks * kKS),
                  ring + (stage % kSA) * ASTAGE + (wave + kWaves * i) * 1024);
    };
    v4i bq[DB][NCF][kKT];
    auto load_b = [&](int slot, int j, int ks) __attribute__((always_inline)) {
        const int f = j / kKT, kt = j % kKT;
        bq[slot][f][kt] = __builtin_amdgcn_raw_buffer_load_b128(brsrc, blane,
                                                                 boff[f] + (ks * kKT + kt) * 1024, 0);
    };

    // ---- A fragment reads: the L limb planes of every row fragment of one K
    // step, read a K step ahead into alternating buffers
    v4i fa[2][L][RF];
    auto read_a = [&](int buf, int stage, int kt) __attribute__((always_inline)) {
#pragma unroll
        for (int rf = 0; rf < RF; ++rf) {
            const int r = 32 * rf + (lane & 31);
            const int c = 2 * kt + (lane >> 5);
            const int8_t* base = ring + (stage % kSA) * ASTAGE + r * kKS + 16 * a_chunk_pos(r, c);
#pragma unroll
            for (int l = 0; l < L; ++l) fa[buf][l][rf] = *reinterpret_cast<const v4i*>(base + l * BM * kKS);
        }
    };

    v16i acc[L][RF][NCF];

    // ---- stream prologue: tile 0's rows and metadata, the A of stages
    // 0 .. kSA-2 and the B of stages 0 .. DB-2 (all of tile 0: nk >= kSA)
    TileInfo cur = info(0);
    fetch_tokens(cur, 0);
    vm_wait<0>();
    lds_barrier();
    fetch_meta(cur, 0);
    make_asrc(cur, 0);
    make_bsrc(cur);
#pragma unroll
    for (int s = 0; s < kSA - 1; ++s)
#pragma unroll
        for (int i = 0; i < APW; ++i) issue_a(i, s, s);
#pragma unroll
    for (int s = 0; s < DB - 1; ++s)
#pragma unroll
        for (int j = 0; j < BPW; ++j) load_b(s, j, s);
    // A(0) landed and published; its first K step's fragments
    vm_wait<0>();
    lds_barrier();
    read_a(0, 0, 0);

    int m = 0;
    int g = 0;  // stage index in the stream
    for (int i = 0; i < tr.ntiles; ++i) {
        const bool has_next = i + 1 < tr.ntiles;
        TileInfo nxt = cur;
        if (has_next) nxt = info(i + 1);
        const int mn = m ^ 1;
        // the stage items load kSA-1 (A) and DB-1 (B) stages ahead: the next
        // tile's sources switch in at these stages of this tile.  Past the
        // end of the stream the items repeat this tile's loads into slots no
        // stage reads (no branch in the load pattern, and the vmcnt counts
        // hold everywhere).
        const int ka_switch = nk - (kSA - 1), kb_switch = nk - (DB - 1);

        // One stage: K steps kt = 0..kKT-1, each the L * RF * NCF MFMAs with
        // the stage's load items spread over its row-fragment groups.  The
        // wait for A(g+1) and the barrier that publishes it come before the
        // last K step, whose MFMAs overlap the reads of the next stage's first
        // K step.
        auto stage = [&](int ks, auto phase, auto first) __attribute__((always_inline)) {
            constexpr int PH = decltype(phase)::value;
            constexpr int WS = PH;                   // B ring slot this stage uses
            constexpr int WL = (PH + DB - 1) % DB;   // slot its B items fill
            const int ta = g + kSA - 1;              // stage its A items load
            const int ksa = ks + kSA - 1 < nk ? ks + kSA - 1 : ks + kSA - 1 - nk;
            const int ksb = ks + DB - 1 < nk ? ks + DB - 1 : ks + DB - 1 - nk;
            if (ks == ka_switch && has_next) {
                // gate/up: the next tile's tokens, fetched after stage 1 of
                // this tile, are visible since the barrier of stage 4
                make_asrc(nxt, mn);
                fetch_meta(nxt, mn);
            }
            if (ks == kb_switch && has_next) make_bsrc(nxt);
            const bool steady = g >= kSA - 2;
#pragma unroll
            for (int kt = 0; kt < kKT; ++kt) {
                if (kt == kKT - 1) {
                    // A(g+1) has landed (stage g+2-kSA issued it); publish it
                    if (steady) vm_wait<T::wait_count>();
                    else vm_wait<0>();
                    lds_barrier();
                }
                const int rb = kt & 1;  // kKT is even: every stage starts on buffer 0
                // the next K step's fragments (after the last: the next
                // stage's first, published by the barrier above)
                if (kt + 1 < kKT) read_a(rb ^ 1, g, kt + 1);
                else read_a(rb ^ 1, g + 1, 0);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int rf = 0; rf < RF; ++rf) {
                    const int gi = kt * RF + rf;
#pragma unroll
                    for (int j = 0; j < NV; ++j) {
                        if (T::item_group(j) == gi) {
                            __builtin_amdgcn_sched_barrier(0);
                            if (T::item_is_a(j)) issue_a(T::item_a(j), ta, ksa);
                            else load_b(WL, T::item_b(j), ksb);
                            __builtin_amdgcn_sched_barrier(0);
                        }
                    }
#pragma unroll
                    for (int l = 0; l < L; ++l)
#pragma unroll
                        for (int f = 0; f < NCF; ++f) {
                            if (decltype(first)::value && kt == 0)
                                acc[l][rf][f] = mfma32(fa[rb][l][rf], bq[WS][f][kt], v16i{});
                            else
                                acc[l][rf][f] = mfma32(fa[rb][l][rf], bq[WS][f][kt], acc[l][rf][f]);
                        }
                }
            }
            // the next tile's tokens, into the buffer the previous tile's
            // sources were made from (every wave is past that: barriers since)
            if (ks == 1 && has_next) fetch_tokens(nxt, mn);
            ++g;
        };

        // stages in groups of DB (static B ring slots); the first stage
        // starts the accumulators
        stage(0, std::integral_constant<int, 0>{}, std::true_type{});
        if constexpr (DB > 1) stage(1, std::integral_constant<int, 1 % DB>{}, std::false_type{});
        if constexpr (DB > 2) stage(2, std::integral_constant<int, 2 % DB>{}, std::false_type{});
        if constexpr (DB > 3) stage(3, std::integral_constant<int, 3 % DB>{}, std::false_type{});
#pragma clang loop unroll(disable)
        for (int ks = DB; ks < nk; ks += DB) {
            stage(ks, std::integral_constant<int, 0>{}, std::false_type{});
            if constexpr (DB > 1) stage(ks + 1, std::integral_constant<int, 1 % DB>{}, std::false_type{});
            if constexpr (DB > 2) stage(ks + 2, std::integral_constant<int, 2 % DB>{}, std::false_type{});
            if constexpr (DB > 3) stage(ks + 3, std::integral_constant<int, 3 % DB>{}, std::false_type{});
        }

        // ---- epilogue (the next tile's first stages are in flight).  The
        // zero-point correction is chosen once per tile (uniform), so no
        // per-element test drags integer multiplies into the common case.
        auto epilogue = [&](auto with_zp) __attribute__((always_inline)) {
            constexpr bool ZP = decltype(with_zp)::value;
            const int e = cur.e;
            const float sa = s_sa[e], sb = s_sb[e];
            const int za = s_za[e], zb = s_zb[e];
            // lane's row within a row quad (0 or 4) and column; everything
            // else is uniform per (row fragment, quad)
            const int lrow = 4 * (lane >> 5);
            float* obase = out + (int64_t)cur.g0 * N + cur.n0 + (GU ? 32 : 64) * wave +
                           (int64_t)lrow * N + (lane & 31);
#pragma unroll
            for (int rf = 0; rf < RF; ++rf) {
                if (32 * rf >= cur.nrows) continue;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int r0 = 32 * rf + 8 * q;          // uniform
                    const int nlive = cur.nrows - r0 - lrow;  // rows t4 < nlive are live
                    const float4 as4 = *reinterpret_cast<const float4*>(&s_as[m][r0 + lrow]);
                    int4 ad4[L];
                    if constexpr (ZP) {
#pragma unroll
                        for (int l = 0; l < L; ++l) ad4[l] = *reinterpret_cast<const int4*>(&s_ad[m][l][r0 + lrow]);
                    }
                    float* o = obase + (int64_t)r0 * N;
#pragma unroll
                    for (int t4 = 0; t4 < 4; ++t4) {
                        const int v = 4 * q + t4;
                        const float asc = t4 == 0 ? as4.x : t4 == 1 ? as4.y : t4 == 2 ? as4.z : as4.w;
                        float val[NCF];
#pragma unroll
                        for (int f = 0; f < NCF; ++f) {
                            int p[L];
#pragma unroll
                            for (int l = 0; l < L; ++l) {
                                p[l] = acc[l][rf][f][v];
                                if constexpr (ZP) {
                                    const int ds = t4 == 0 ? ad4[l].x : t4 == 1 ? ad4[l].y : t4 == 2 ? ad4[l].z : ad4[l].w;
                                    p[l] -= (GU && f == 1 ? zb : za) * ds;
                                }
                            }
                            const float wsc = __fmul_rn(asc, GU && f == 1 ? sb : sa);
                            val[f] = __fmul_rn(hm_recombine(p, L), wsc);
                        }
                        if constexpr (GU) {
                            // z = silu(g) * u (Activation.cpp:44, then the multiply)
                            const float z = __fmul_rn(hm_silu_t(val[0], s_exp2), val[1]);
                            if (t4 < nlive) o[(int64_t)t4 * N] = z;
                        } else {
                            if (t4 < nlive) {
                                o[(int64_t)t4 * N] = val[0];
                                o[(int64_t)t4 * N + 32] = val[1];
                            }
                        }
                    }
                    // one (row fragment, row quad) at a time: the scheduler
                    // would otherwise start every group's accumulator reads
                    // and exponentials at once and spill
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        };
        const bool zpt = GU ? ((s_za[cur.e] | s_zb[cur.e]) != 0) : (s_za[cur.e] != 0);
        if (zpt) epilogue(std::true_type{});
        else epilogue(std::false_type{});
        m = mn;
        cur = nxt;
    }
    vm_wait<0>();
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

// B ring depth for nk stages per tile: the largest of 4, 3, 2 dividing nk.
int ring_depth(int64_t nk) { return nk % 4 == 0 ? 4 : nk % 3 == 0 ? 3 : nk % 2 == 0 ? 2 : 0; }

bool shape_ok(int role, int64_t K, int64_t N, int64_t E, int32_t limbs) {
    // |P_l| <= K * 128 * 255 < 2^31 keeps every limb partial exact: K <= 65536
    if (limbs < 1 || limbs > 3 || E < 1 || E > kMaxExperts || K > 65536 || N > (1 << 20))
        return false;
    if (K % kKS != 0) return false;
    const int64_t nk = K / kKS;
    const int64_t bn = role == kGateUp ? 32 * kWaves : 64 * kWaves;
    // gate/up reads the next tile's tokens (fetched after stage 1) from
    // stage 4 on and needs them kSA - 1 stages before the tile ends
    const int64_t min_nk = role == kGateUp ? 2 * kSA : kSA;
    return nk >= min_nk && ring_depth(nk) != 0 && N % bn == 0;
}

template <int ROLE, int L, int DB>
int launch(const hm_layer* layer, const int8_t* adig, const float* ascale, const int32_t* adsum,
           int64_t arows, const int32_t* counts, const int32_t* offsets,
           const int32_t* perm_tokens, float* out, bool timed, hipStream_t stream) {
    const int64_t H = layer->hidden, I = layer->intermediate;
    const int64_t K = ROLE == kGateUp ? H : I, N = ROLE == kGateUp ? I : H;
    // buffer offsets are 32-bit: the digit planes and one expert's tiles
    if ((int64_t)L * arows * K > INT_MAX || 3 * hm_proj_bytes(H, I) > INT_MAX || arows > INT_MAX)
        return HM_ERR_UNSUPPORTED;
    HM_STAGE_LAUNCH(timed, false, (limb_gemm_kernel<ROLE, L, DB>), dim3((unsigned)persistent_grid()),
                    dim3(kThreads), 0, stream, adig, ascale, adsum, (int)arows, (int)K, (int)N,
                    (int)H, (int)I, (int)layer->experts, static_cast<const int8_t*>(layer->packed),
                    layer->scale, layer->zero_point, counts, offsets, perm_tokens, out);
    HM_LAUNCHED();
    return HM_OK;
}

template <int ROLE, int L>
int launch_l(const hm_layer* layer, const int8_t* adig, const float* ascale,
             const int32_t* adsum, int64_t arows, const int32_t* counts, const int32_t* offsets,
             const int32_t* perm_tokens, float* out, bool timed, hipStream_t stream) {
    const int64_t K = ROLE == kGateUp ? layer->hidden : layer->intermediate;
    switch (ring_depth(K / kKS)) {
    case 4: return launch<ROLE, L, 4>(layer, adig, ascale, adsum, arows, counts, offsets, perm_tokens, out, timed, stream);
    case 3: return launch<ROLE, L, 3>(layer, adig, ascale, adsum, arows, counts, offsets, perm_tokens, out, timed, stream);
    case 2: return launch<ROLE, L, 2>(layer, adig, ascale, adsum, arows, counts, offsets, perm_tokens, out, timed, stream);
    default: return HM_ERR_UNSUPPORTED;
    }
}

}  // namespace

// Shape preconditions of the MFMA kernels: K in 128-byte stages (enough of
// them for the stream's look-ahead, a count the B register ring divides),
// N in whole workgroup column blocks, E <= 256 (tables in LDS).
bool hm_mfma_gateup_ok(int64_t H, int64_t I, int64_t E, int32_t limbs) {
    return shape_ok(kGateUp, H, I, E, limbs);
}

bool hm_mfma_down_ok(int64_t H, int64_t I, int64_t E, int32_t limbs) {
    return shape_ok(kDown, I, H, E, limbs);
}

// zf [R x I]: z = silu(g) * u of every grouped row.  The first kernel of the
// gate/up stage (its start opens an armed stage timer).
int hm_launch_gateup_i8_mfma(const hm_layer* layer, int32_t limbs, const int8_t* xdig,
                             const float* xscale, const int32_t* xdsum, int64_t tokens,
                             const int32_t* counts, const int32_t* offsets,
                             const int32_t* perm_tokens, int64_t R, float* zf,
                             hipStream_t stream) {
    if (tokens > INT_MAX || R > INT_MAX) return HM_ERR_OVERFLOW;
    switch (limbs) {
    case 1: return launch_l<kGateUp, 1>(layer, xdig, xscale, xdsum, tokens, counts, offsets, perm_tokens, zf, true, stream);
    case 2: return launch_l<kGateUp, 2>(layer, xdig, xscale, xdsum, tokens, counts, offsets, perm_tokens, zf, true, stream);
    case 3: return launch_l<kGateUp, 3>(layer, xdig, xscale, xdsum, tokens, counts, offsets, perm_tokens, zf, true, stream);
    default: return HM_ERR_INVALID;
    }
}

// y [R x H] from the Z digit planes [L][R][I] (one scale per row).
int hm_launch_down_i8_mfma(const hm_layer* layer, int32_t limbs, const int32_t* counts,
                           const int32_t* offsets, int64_t R, const int8_t* zdig,
                           const float* zscale, const int32_t* zdsum, float* y,
                           hipStream_t stream) {
    if (R > INT_MAX) return HM_ERR_OVERFLOW;
    switch (limbs) {
    case 1: return launch_l<kDown, 1>(layer, zdig, zscale, zdsum, R, counts, offsets, nullptr, y, false, stream);
    case 2: return launch_l<kDown, 2>(layer, zdig, zscale, zdsum, R, counts, offsets, nullptr, y, false, stream);
    case 3: return launch_l<kDown, 3>(layer, zdig, zscale, zdsum, R, counts, offsets, nullptr, y, false, stream);
    default: return HM_ERR_INVALID;
    }
}
