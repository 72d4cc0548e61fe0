// hm_gemm_mfma.hip -- grouped INT8-MFMA expert GEMMs for gfx950.
//
// The activation operand is L fixed-point digit planes with one scale per
// row (hm_device.h); every plane meets the same weight fragment in one
// v_mfma_i32_32x32x32_i8, so each plane's int32 partial over the whole row
// is exact, and the epilogues recombine them (hm_recombine) exactly as the
// generic kernels and the CPU restatement do.  Weights are 1 KB tiles in
// MFMA B-operand order (hm_tile_offset): one 16-byte-per-lane load of a
// contiguous kilobyte is one B fragment.
//
// Operand layout of v_mfma_i32_32x32x32_i8: lane l supplies 16 bytes of row
// l % 32 of A and of column l % 32 of B, K bytes 16 (l / 32) .. +15 of the
// 32-wide step; its 16 int32 results are column l % 32, rows
// 8 (v / 4) + 4 (l / 32) + v % 4 (v = 0..15).
//
// Persistent kernels, one workgroup per CU:
//   ring_gemm_kernel<L, false> (gate/up): 8 wave64s (two per SIMD), A (the
//            token rows' X digit planes, gathered by perm_tokens) and B both
//            staged through an LDS ring by DMA; epilogue g and u -> floats
//            (the SwiGLU runs in the Z quantisation pass, hm_gemm.hip).
//   ring_gemm_kernel<L, true> (down): the same kernel on the grouped rows'
//            Z digit planes and the down tiles; epilogue y -> floats.
//   limb_gemm_kernel (down, for shapes the ring does not take): 4 wave64s
//            (one per SIMD, 512 registers: the accumulators take the
//            AGPRs), A through an LDS ring by DMA, B straight into a
//            register ring.
//
// limb_gemm_kernel, per stage of K = 128 bytes (four MFMA K steps):
//   A  global -> LDS by 16-byte buffer loads to LDS (inline asm), 128-byte
//      row chunks (whole cache lines), into a ring of kSA stages.  Each row's
//      eight 16-byte chunks are stored rotated by (row >> 1) & 7, so the
//      readers' ds_read_b128 over any 16 lanes hit 16 distinct bank groups.
//   B  global -> VGPRs, a ring of DB stages of registers, loaded DB-1 stages
//      ahead by loads the compiler does not track (buf_load16).
// One vmcnt wait per stage completes both operands of the next stage.
// Every wave issues its share of the loads of later stages between the
// MFMAs of the current one (a wave that issues its loads in a clump stalls
// the matrix pipe behind them).  Stages form one stream per workgroup across
// its tiles, so the next tile's first stages load during the current tile's
// last stages and its epilogue.  The kernel waits for its loads with
// explicit vmcnt counts (every vector memory instruction between the awaited
// load and the wait is counted; stores and metadata loads only add to the
// count, which keeps the wait conservative).  A tile is BM grouped rows of
// one expert x 256 output columns; every wave holds all BM rows and its own
// two 32-column fragments (output columns 64 w .. +63).
//
// Tile order (both kernels): tiles are numbered m-tile major, column block
// minor, and split into 8 contiguous ranges, one per XCD (workgroup i runs
// on XCD i % 8), so the column blocks of an m-tile (sharing A rows) and the
// m-tiles of one expert (sharing B tiles) meet in one XCD's L2.  In an
// expert's partial last tile, the 32-row fragments past its last row skip
// their MFMAs (down: tiles of two row fragments; gate/up: the waves whose
// rows all lie past it).
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

template <int L, int DB>
struct Tile {
    static constexpr int RF = L <= 2 ? 4 : 2;            // 32-row fragments per tile
    static constexpr int BM = 32 * RF;                   // tile rows
    static constexpr int NCF = 2;                        // 32-column fragments per wave
    static constexpr int BN = 32 * NCF * kWaves;             // output columns
    static constexpr int ASTAGE = L * BM * kKS;          // A bytes per stage
    static constexpr int ALOADS = ASTAGE / 1024;         // wave-wide A loads per stage
    static constexpr int APW = ALOADS / kWaves;          // ... per wave
    static constexpr int BPW = NCF * kKT;                // B loads per wave per stage
    static constexpr int NV = APW + BPW;                 // loads per wave per stage
    static constexpr int NG = kKT * RF;                  // (K step, row fragment) groups per stage
    static_assert(ALOADS % kWaves == 0 && APW <= BPW && DB >= 2 && DB <= kSA && kKT % 2 == 0,
                  "tile shape");
    // A stage's load items: its B loads first, then its A DMAs; item j is
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
    static_assert(item_group(BPW - 1) < kWaitGroup, "B items precede the wait");
    // The one wait of stage g completes both operands of stage g+1:
    //   A(g+1): DMAs of stage g+2-kSA, the last items of that stage;
    //   B(g+1): loads of stage g+2-DB, the first BPW items of that stage.
    // Each count is the number of loads issued after the last awaited one
    // (vector memory loads complete in issue order).
    static constexpr int a_count = (kSA - 3) * NV + items_before(kWaitGroup);
    static constexpr int b_count = (DB - 2) * NV + items_before(kWaitGroup) - BPW;
    static constexpr int wait_count = a_count < b_count ? a_count : b_count;
    static_assert(wait_count >= 0 && wait_count <= 63, "vmcnt");
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

// One wave-wide 16-byte buffer -> VGPR load the compiler does not track:
// it inserts no wait for the result, so the kernel's own vmcnt waits (which
// count the DMAs too) decide when the registers are complete, and
// publish() marks that point.  (The compiler's own waits would count only
// the loads it knows of and so drain loads issued half as long ago as the
// register ring allows.)  Until its wait the register must not be read,
// copied or spilled; the build checks this on the compiled code, along every
// control-flow path (hmoe/isa_check.py), and refuses a library that breaks it.
__device__ __forceinline__ v4i buf_load16(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff, uint32_t soff) {
    v4i r;
    asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(r) : "v"(voff), "s"(rsrc), "s"(soff));
    return r;
}
// After the vmcnt wait that completes a buf_load16: ties the value to that
// point, so no use of it is scheduled before the wait.
__device__ __forceinline__ void publish(v4i& r) { asm volatile("" : "+v"(r)); }

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
// Experts with at most `skinny` rows get no tiles (skinny_split_kernel
// takes them).
__device__ __forceinline__ void tile_prefix(const int32_t* cnt, int E, int bm, int skinny,
                                            int32_t* prefix) {
    const int lane = threadIdx.x & (HM_WAVE - 1);
    int base = 0;
    for (int c0 = 0; c0 < E; c0 += HM_WAVE) {
        const int e = c0 + lane;
        const int n = e < E && cnt[e] > skinny ? (cnt[e] + bm - 1) / bm : 0;
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
// The down projection: K = I, N = H, out = y [R x H].  A rows: the Z digit
// planes adig (the Z layout hm_dlay_z: [K/64][L][R][64]) by grouped row;
// ascale/adsum: their fixed-point scales [arows] and digit sums [L][arows]
// (for non-zero zero points).
// ---------------------------------------------------------------------------
template <int L, int DB>
__global__ __launch_bounds__(kThreads) void limb_gemm_kernel(
    const int8_t* __restrict__ adig, const float* __restrict__ ascale,
    const int32_t* __restrict__ adsum, int arows, int K, int N, int H, int I, int experts,
    const int8_t* __restrict__ packed, const float* __restrict__ scale,
    const int32_t* __restrict__ zp, const int32_t* __restrict__ counts,
    const int32_t* __restrict__ offsets, int skinny, float* __restrict__ out) {
    using T = Tile<L, DB>;
    constexpr int RF = T::RF, BM = T::BM, BN = T::BN, NCF = T::NCF, APW = T::APW,
                  BPW = T::BPW, NV = T::NV, ASTAGE = T::ASTAGE;
    constexpr int MW = BM / HM_WAVE;  // 64-row metadata chunks of a tile
    __shared__ __attribute__((aligned(1024))) int8_t ring[kSA * ASTAGE];
    __shared__ int32_t s_prefix[kMaxExperts + 1];
    __shared__ int32_t s_off[kMaxExperts], s_cnt[kMaxExperts];
    __shared__ float s_sa[kMaxExperts];     // down projection scale
    __shared__ int32_t s_za[kMaxExperts];   // and zero point
    __shared__ __attribute__((aligned(16))) float s_as[2][BM];       // A row scale
    __shared__ __attribute__((aligned(16))) int32_t s_ad[2][L][BM];  // A row digit sums

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int E = experts;
    for (int e = tid; e < E; e += kThreads) {
        s_cnt[e] = counts[e];
        s_off[e] = offsets[e];
        s_sa[e] = scale[3 * e + 2];
        s_za[e] = zp[3 * e + 2];
    }
    __syncthreads();
    if (wave == 0) tile_prefix(s_cnt, E, BM, skinny, s_prefix);
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
    // the A rows' scales and digit sums into s_as[m], s_ad[m]
    auto fetch_meta = [&](const TileInfo& t, int m) __attribute__((always_inline)) {
        if (wave < MW) {
            const int r = HM_WAVE * wave + fresh_lane();
            const int src = t.g0 + min(r, t.nrows - 1);
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
    // which holds chunk a_chunk_pos(row, lane%8) of the row's stage: in the Z
    // layout, 16-byte piece c of stage ks lies in 64-byte chunk 2 ks + c/4
    // (the stage's uniform offset ks * astep, astep = 2 L arows 64).
    const __amdgpu_buffer_rsrc_t arsrc = buffer_rsrc(adig, (uint32_t)((int64_t)L * arows * K));
    const uint32_t astep = (uint32_t)(2 * 64 * (int64_t)L * arows);
    uint32_t aoff[APW];
    auto make_asrc = [&](const TileInfo& t) __attribute__((always_inline)) {
        const int ln = fresh_lane();
#pragma unroll
        for (int i = 0; i < APW; ++i) {
            const int q = 8 * (wave + kWaves * i) + (ln >> 3);
            const int l = q / BM, r = q % BM;
            const int c = a_chunk_pos(r, ln & 7);
            const int row = t.g0 + min(r, t.nrows - 1);
            aoff[i] = (uint32_t)((((int64_t)(c >> 2) * L + l) * arows + row) * 64 + 16 * (c & 3));
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
            const int cb = t.n0 / 32 + NCF * wave + f;
            boff[f] = (int)(2 * hm_proj_bytes(H, I) + (int64_t)cb * (K32 / 32) * 1024);
        }
    };
    auto issue_a = [&](int i, int stage, int ks) __attribute__((always_inline)) {
        dma16_buf(arsrc, aoff[i], (uint32_t)ks * astep,
                  ring + (stage % kSA) * ASTAGE + (wave + kWaves * i) * 1024);
    };
    v4i bq[DB][NCF][kKT];
    auto publish_slot = [&](int slot) __attribute__((always_inline)) {
#pragma unroll
        for (int f = 0; f < NCF; ++f)
#pragma unroll
            for (int kt = 0; kt < kKT; ++kt) publish(bq[slot][f][kt]);
    };
    auto load_b = [&](int slot, int j, int ks) __attribute__((always_inline)) {
        const int f = j / kKT, kt = j % kKT;
        bq[slot][f][kt] = buf_load16(brsrc, blane, (uint32_t)(boff[f] + (ks * kKT + kt) * 1024));
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

    // ---- stream prologue: tile 0's row metadata, the A of stages 0 .. kSA-2
    // and the B of stages 0 .. DB-2 (all of tile 0: nk >= kSA)
    TileInfo cur = info(0);
    fetch_meta(cur, 0);
    make_asrc(cur);
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
#pragma unroll
    for (int s = 0; s < DB - 1; ++s) publish_slot(s);
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
                make_asrc(nxt);
                fetch_meta(nxt, mn);
            }
            if (ks == kb_switch && has_next) make_bsrc(nxt);
#pragma unroll
            for (int kt = 0; kt < kKT; ++kt) {
                if (kt == kKT - 1) {
                    // A(g+1) and B(g+1) have landed (issued by stages
                    // g+2-kSA and g+2-DB, or by the prologue, which ends with
                    // a full wait); the barrier publishes A(g+1)
                    vm_wait<T::wait_count>();
                    lds_barrier();
                    publish_slot((PH + 1) % DB);
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
                    // row fragments past the tile's last row (an expert's
                    // partial last tile) skip their MFMAs; the epilogue skips
                    // their accumulators.  Only with two row fragments: with
                    // four, the branches split the accumulator ranges and the
                    // allocator spills them.
                    if (RF <= 2 ? (rf == 0 || 32 * rf < cur.nrows) : true) {
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
            }
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
            const float sa = s_sa[e];
            const int za = s_za[e];
            // out [R x N], the wave's two fragments side by side.  The
            // lane's row within a row quad (0 or 4) and its column;
            // everything else is uniform per (row fragment, quad).
            const int64_t ldo = N;
            const int fstride = 32;
            const int lrow = 4 * (lane >> 5);
            float* obase = out + (int64_t)cur.g0 * ldo + cur.n0 + 64 * wave +
                           (int64_t)lrow * ldo + (lane & 31);
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
                    float* o = obase + (int64_t)r0 * ldo;
#pragma unroll
                    for (int t4 = 0; t4 < 4; ++t4) {
                        const int v = 4 * q + t4;
                        const float asc = t4 == 0 ? as4.x : t4 == 1 ? as4.y : t4 == 2 ? as4.z : as4.w;
                        if (t4 < nlive) {
#pragma unroll
                            for (int f = 0; f < NCF; ++f) {
                                int p[L];
#pragma unroll
                                for (int l = 0; l < L; ++l) {
                                    p[l] = acc[l][rf][f][v];
                                    if constexpr (ZP) {
                                        const int ds = t4 == 0 ? ad4[l].x : t4 == 1 ? ad4[l].y : t4 == 2 ? ad4[l].z : ad4[l].w;
                                        p[l] -= za * ds;
                                    }
                                }
                                const float wsc = __fmul_rn(asc, sa);
                                o[(int64_t)t4 * ldo + fstride * f] = __fmul_rn(hm_recombine(p, L), wsc);
                            }
                        }
                    }
                    // one (row fragment, row quad) at a time: the scheduler
                    // would otherwise start every group's accumulator reads
                    // at once and spill
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        };
        const bool zpt = s_za[cur.e] != 0;
        if (zpt) epilogue(std::true_type{});
        else epilogue(std::false_type{});
        m = mn;
        cur = nxt;
    }
    vm_wait<0>();
}

// ===========================================================================
// Skinny groups: bounded split-K.  An expert with at most kSkinnyRows = 32
// grouped rows (a cold expert; most experts of a mid-size batch) would
// fill a tile of BM rows mostly with padding, and the tile still streams
// every row of its A stages.  Such experts skip the tile kernels
// (tile_prefix) and come here: one workgroup per (expert, kSkCB column
// blocks of 32); its A rows (all K, the L digit planes) go to LDS once, in
// MFMA operand order, and its 8 waves are kSkCB column blocks x kSkP K
// parts.  Each wave streams its block's weight tiles over its K part and
// runs v_mfma_i32_32x32x32_i8 on its own accumulators; the parts' int32
// limb partials meet in LDS in part order (integer addition: exact, so the
// partials, and hence the epilogue's floats, equal the tile kernels' bit
// for bit).  K is split into a bounded number of parts as the reference's
// split-K does (P = min(8, ceil(K/512)), Int8GemmPlan.cpp:29-53, reduced in
// a fixed order, CudaKernels.cu:53-107), here kSkP = 2 within a workgroup.
//   GU    gate and up (NP = 2): A = the X digit planes of the rows' tokens
//         (perm_tokens; hm_dlay_x), out = gu [R x 2I];
//   down  (NP = 1): A = the Z digit planes of the grouped rows (hm_dlay_z),
//         out = y.
// LDS: the A rows, L x 32 x K bytes, reused for the partials (skinny_lds).
// ===========================================================================
constexpr int kSkinnyRows = 32;   // one 32-row fragment
constexpr int kSkWaves = 8;
constexpr int kSkThreads = 64 * kSkWaves;
constexpr int kSkP = 2;           // K parts
constexpr int kSkCB = kSkWaves / kSkP;  // column blocks per workgroup
constexpr int kSkLds = 131072;    // A bytes in LDS: L * 32 * K
constexpr int kSkDepth = 4;       // K steps of weights in flight per wave

template <int L, bool GU>
__global__ __launch_bounds__(kSkThreads) void skinny_split_kernel(
    const int8_t* __restrict__ adig, const float* __restrict__ ascale,
    const int32_t* __restrict__ adsum, int arows, const int32_t* __restrict__ perm_tokens,
    int K, int N, int H, int I, const int8_t* __restrict__ packed,
    const float* __restrict__ scale, const int32_t* __restrict__ zp,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    float* __restrict__ out) {
    constexpr int NP = GU ? 2 : 1;
    extern __shared__ __attribute__((aligned(1024))) int8_t s_a[];   // [L][KT][32 rows][32 B]
    __shared__ int32_t s_arow[32];
    const int e = blockIdx.y;
    const int nrows = counts[e];
    if (nrows == 0 || nrows > kSkinnyRows) return;          // (uniform)
    const int g0 = offsets[e];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int KT = K / 32;
    if (tid < 32) {
        const int g = g0 + min(tid, nrows - 1);  // rows past the group repeat its last
        s_arow[tid] = GU ? perm_tokens[g] : g;
    }
    __syncthreads();
    // the A rows into LDS: one wave-wide 16-byte load per (plane, K step):
    // lane -> row lane/2, half lane%2 (32 rows x 32 bytes, MFMA order)
    {
        const int arow = s_arow[lane >> 1];
        const hm_dlay lay = GU ? hm_dlay_x(L, K) : hm_dlay_z(L, arows);
        for (int q = wave; q < L * KT; q += kSkWaves) {
            const int l = q / KT, kt = q - l * KT;
            dma16(adig + hm_dlay_off(lay, l, arow, 32 * kt + 16 * (lane & 1)), s_a + 1024 * q);
        }
    }
    // this wave's column block and K part
    const int cbl = wave % kSkCB, part = wave / kSkCB;
    const int cb = blockIdx.x * kSkCB + cbl;                // output columns 32 cb .. +31
    const int kt0 = part * KT / kSkP, kt1 = (part + 1) * KT / kSkP;
    const bool live = 32 * cb < N;                          // (uniform per wave)
    const int8_t* bsrc[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p)
        bsrc[p] = packed + hm_proj_offset(e, GU ? p : 2, H, I) +
                  (int64_t)min(cb, N / 32 - 1) * KT * 1024 + 16 * lane;
    // weights kSkDepth steps ahead (a step past the part re-reads its last)
    v4i fb[kSkDepth][NP];
#pragma unroll
    for (int d = 0; d < kSkDepth; ++d)
#pragma unroll
        for (int p = 0; p < NP; ++p)
            fb[d][p] = *reinterpret_cast<const v4i*>(bsrc[p] + (int64_t)min(kt0 + d, kt1 - 1) * 1024);
    vm_wait<0>();   // this wave's A loads (the first weights land about as soon)
    lds_barrier();  // every wave's
    v16i acc[L][NP];
#pragma unroll
    for (int l = 0; l < L; ++l)
#pragma unroll
        for (int p = 0; p < NP; ++p) acc[l][p] = v16i{};
    const int aoff = 32 * (lane & 31) + 16 * (lane >> 5);
    for (int kt = kt0; kt < kt1; kt += kSkDepth) {
#pragma unroll
        for (int d = 0; d < kSkDepth; ++d) {
            if (kt + d < kt1) {
                v4i fa[L];
#pragma unroll
                for (int l = 0; l < L; ++l)
                    fa[l] = *reinterpret_cast<const v4i*>(s_a + 1024 * (l * KT + kt + d) + aoff);
#pragma unroll
                for (int l = 0; l < L; ++l)
#pragma unroll
                    for (int p = 0; p < NP; ++p) acc[l][p] = mfma32(fa[l], fb[d][p], acc[l][p]);
            }
#pragma unroll
            for (int p = 0; p < NP; ++p)
                fb[d][p] = *reinterpret_cast<const v4i*>(
                    bsrc[p] + (int64_t)min(kt + d + kSkDepth, kt1 - 1) * 1024);
        }
    }
    // the parts' partials meet in LDS (the A copy is no longer read)
    __syncthreads();
    int32_t* s_p = reinterpret_cast<int32_t*>(s_a);          // [part-1][cbl][L][NP][16][64]
    constexpr int PW = L * NP * 16 * HM_WAVE;                // ints per wave
    if (part > 0) {
#pragma unroll
        for (int l = 0; l < L; ++l)
#pragma unroll
            for (int p = 0; p < NP; ++p)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    s_p[((part - 1) * kSkCB + cbl) * PW + ((l * NP + p) * 16 + v) * HM_WAVE + lane] = acc[l][p][v];
    }
    __syncthreads();
    if (part > 0 || !live) return;
#pragma unroll
    for (int q = 1; q < kSkP; ++q)
#pragma unroll
        for (int l = 0; l < L; ++l)
#pragma unroll
            for (int p = 0; p < NP; ++p)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    acc[l][p][v] += s_p[((q - 1) * kSkCB + cbl) * PW + ((l * NP + p) * 16 + v) * HM_WAVE + lane];
    // epilogue, as the tile kernels': result register v of lane m is row
    // 8 (v/4) + 4 (m/32) + v%4, column m%32
    const int zpa = zp[3 * e + (GU ? 0 : 2)], zpb = GU ? zp[3 * e + 1] : 0;
    const float sa = scale[3 * e + (GU ? 0 : 2)], sb = GU ? scale[3 * e + 1] : 0.0f;
    const int64_t n = 32 * (int64_t)cb + (lane & 31);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int row = 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (row >= nrows) continue;
        const int arow = s_arow[row];
        const float asc = ascale[arow];
        int pa[L], pb[L];
#pragma unroll
        for (int l = 0; l < L; ++l) {
            pa[l] = acc[l][0][v];
            pb[l] = acc[l][NP - 1][v];
        }
        if (zpa != 0 || zpb != 0) {
#pragma unroll
            for (int l = 0; l < L; ++l) {
                const int ds = adsum[(int64_t)l * arows + arow];
                pa[l] -= zpa * ds;
                pb[l] -= zpb * ds;
            }
        }
        if (GU) {
            const float fg = __fmul_rn(asc, sa), fu = __fmul_rn(asc, sb);
            float* grow = out + (int64_t)(g0 + row) * (2 * (int64_t)I) + n;
            grow[0] = __fmul_rn(hm_recombine(pa, L), fg);
            grow[I] = __fmul_rn(hm_recombine(pb, L), fu);
        } else {
            out[(int64_t)(g0 + row) * N + n] = __fmul_rn(hm_recombine(pa, L), __fmul_rn(asc, sa));
        }
    }
}

// Dynamic LDS of the skinny kernel: the A rows, or the K parts' partials
// (parts 1 .. kSkP-1, 16 ints per lane per accumulator) if larger.
size_t skinny_lds(int64_t K, int32_t limbs, bool gu) {
    const size_t a = (size_t)limbs * 32 * K;
    const size_t p = (size_t)(kSkP - 1) * kSkCB * limbs * (gu ? 2 : 1) * 16 * HM_WAVE * sizeof(int32_t);
    return a > p ? a : p;
}

// Whether the skinny kernel takes this projection: its LDS fits and K
// splits into whole K steps.
bool skinny_ok(int64_t K, int64_t N, int32_t limbs, bool gu) {
    return skinny_lds(K, limbs, gu) <= (size_t)kSkLds && K % 32 == 0 && K / 32 >= kSkP &&
           N % 32 == 0;
}

template <int L, bool GU>
int launch_skinny(const hm_layer* layer, const int8_t* adig, const float* ascale,
                  const int32_t* adsum, int64_t arows, const int32_t* perm_tokens,
                  const int32_t* counts, const int32_t* offsets, float* out, hipStream_t stream,
                  bool timed_first) {
    const int64_t H = layer->hidden, I = layer->intermediate;
    const int64_t K = GU ? H : I, N = GU ? I : H;
    const dim3 grid((unsigned)((N / 32 + kSkCB - 1) / kSkCB), (unsigned)layer->experts);
    const size_t lds = skinny_lds(K, L, GU);
    HM_STAGE_LAUNCH(timed_first, false, (skinny_split_kernel<L, GU>), grid, dim3(kSkThreads), lds,
                    stream, adig, ascale, adsum, (int)arows, perm_tokens, (int)K, (int)N, (int)H,
                    (int)I, static_cast<const int8_t*>(layer->packed), layer->scale,
                    layer->zero_point, counts, offsets, out);
    HM_LAUNCHED();
    return HM_OK;
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

bool shape_ok(int64_t K, int64_t N, int64_t E, int32_t limbs) {
    // |P_l| <= K * 128 * 255 < 2^31 keeps every limb partial exact: K <= 65536
    if (limbs < 1 || limbs > 3 || E < 1 || E > kMaxExperts || K > 65536 || N > (1 << 20))
        return false;
    if (K % kKS != 0) return false;
    const int64_t nk = K / kKS;
    return nk >= kSA && ring_depth(nk) != 0 && N % (64 * kWaves) == 0;
}

template <int L, int DB>
int launch(const hm_layer* layer, const int8_t* adig, const float* ascale, const int32_t* adsum,
           int64_t arows, const int32_t* counts, const int32_t* offsets, int skinny, float* out,
           hipStream_t stream) {
    const int64_t H = layer->hidden, I = layer->intermediate;
    const int64_t K = I, N = H;
    // buffer offsets are 32-bit: the digit planes and one expert's tiles
    if ((int64_t)L * arows * K > INT_MAX || 3 * hm_proj_bytes(H, I) > INT_MAX || arows > INT_MAX)
        return HM_ERR_UNSUPPORTED;
    hipLaunchKernelGGL((limb_gemm_kernel<L, DB>), dim3((unsigned)persistent_grid()), dim3(kThreads), 0,
                       stream, adig, ascale, adsum, (int)arows, (int)K, (int)N, (int)H, (int)I,
                       (int)layer->experts, static_cast<const int8_t*>(layer->packed), layer->scale,
                       layer->zero_point, counts, offsets, skinny, out);
    HM_LAUNCHED();
    return HM_OK;
}

template <int L>
int launch_l(const hm_layer* layer, const int8_t* adig, const float* ascale,
             const int32_t* adsum, int64_t arows, const int32_t* counts, const int32_t* offsets,
             float* out, bool split_k, hipStream_t stream) {
    if (!shape_ok(layer->intermediate, layer->hidden, layer->experts, L) ||
        ring_depth(layer->intermediate / kKS) == 0)
        return HM_ERR_UNSUPPORTED;
    // skinny groups (split K, when asked for), then the tiles of the others
    const bool sk = split_k && skinny_ok(layer->intermediate, layer->hidden, L, false);
    if (sk) {
        const int rc = launch_skinny<L, false>(layer, adig, ascale, adsum, arows, nullptr, counts,
                                               offsets, out, stream, false);
        if (rc) return rc;
    }
    const int skinny = sk ? kSkinnyRows : 0;
    switch (ring_depth(layer->intermediate / kKS)) {
    case 4: return launch<L, 4>(layer, adig, ascale, adsum, arows, counts, offsets, skinny, out, stream);
    case 3: return launch<L, 3>(layer, adig, ascale, adsum, arows, counts, offsets, skinny, out, stream);
    case 2: return launch<L, 2>(layer, adig, ascale, adsum, arows, counts, offsets, skinny, out, stream);
    default: return HM_ERR_UNSUPPORTED;
    }
}

// ===========================================================================
// gate/up: a ring kernel of its own.  8 wave64s per workgroup (two per
// SIMD, 256 registers each), both operands staged through LDS by DMA, so
// while one wave of a SIMD waits (for a stage, or in its epilogue) the other
// keeps the matrix pipe busy.  Tile = BM grouped rows x (128 gate + 128 up)
// weight columns; wave (wr, wc) owns rows [32 WR wr, +32 WR) and gate and up
// columns [32 WCP wc, +32 WCP).  Per ring stage of 64 K bytes:
//   A  the L digit planes of the tile rows (gathered by perm_tokens), in
//      fragments of 32 rows x 64 bytes, two wave-wide 16-byte DMAs each
//      (lane: row 16 h + lane/4, chunk (lane%4) ^ ((lane/16)%4)), read back
//      bank-conflict free with the swizzle of gu_frag_read_offset; at two
//      planes (gate/up) each DMA instead moves 8 rows' whole 128-byte lines
//      (both planes of the stage, adjacent in the X layout) and the reads
//      follow gu_pair_read_offset;
//   B  the 8 weight fragments (4 gate, 4 up column blocks of 32), each the
//      two 1 KB operand-order tiles (hm_tile_offset) of the stage's K steps,
//      one contiguous DMA each and read back at 16 lane.
// The stage's loads are spread over the waves, LPW per wave (the last
// round only on the waves it reaches); a step refills the slot read two
// steps earlier, so its barrier leaves the previous step's fragment reads
// in flight (the K loop below).
// Epilogue: the dequantised g and u values (z = silu(g) * u and the Z digits
// follow in one pass over the rows at full occupancy, hm_gemm.hip).
// ===========================================================================
constexpr int kGuWaves = 8;
constexpr int kGuThreads = 64 * kGuWaves;
constexpr int kGuKB = 64;                   // K bytes per ring stage: two MFMA K steps
constexpr int kGuStages = 4;                // ring stages
constexpr int kGuFrag = 32 * kGuKB;         // bytes of one fragment of a stage
constexpr int kGuN = 128;                   // columns per projection per tile

__device__ __forceinline__ int gu_frag_load_row(int lane, int hf) { return 16 * hf + (lane >> 2); }
__device__ __forceinline__ int gu_frag_load_chunk(int lane) { return (lane & 3) ^ ((lane >> 4) & 3); }
// A fragment reader of K step h: lane m (row r = m%32, chunk c = 2h + m/32)
// at 1024 (r/16) + 16 (4 (r%16) + (c ^ ((r/4)%4))); over any 16 consecutive
// lanes these are 16 distinct 16-byte bank groups.
__device__ __forceinline__ int gu_frag_read_offset(int lane, int h) {
    const int r = lane & 31, c = 2 * h + (lane >> 5);
    return 1024 * (r >> 4) + 16 * (4 * (r & 15) + (c ^ ((r >> 2) & 3)));
}
// The paired (L = 2, gate/up) fragment reader: plane l, K step h, lane m
// (row r = m%32, 16-byte piece c = 4 l + 2 h + m/32 of the row's 128 bytes)
// at 128 r + 16 (c ^ ((r/2)%8)) in the 32-row block; over any 16
// consecutive lanes these are 16 distinct 16-byte bank groups.
__device__ __forceinline__ int gu_pair_read_offset(int lane, int h, int l) {
    const int r = lane & 31, c = 4 * l + 2 * h + (lane >> 5);
    return 128 * r + 16 * (c ^ ((r >> 1) & 7));
}
__device__ __forceinline__ v4i lds16(const int8_t* p) { return *reinterpret_cast<const v4i*>(p); }

template <int L>
struct GateUpTile {
    static constexpr int WR = 1;                        // 32-row fragments per wave
    static constexpr int WCP = L >= 3 ? 1 : 2;          // gate (and up) fragments per wave
    static constexpr int NWC = kGuN / 32 / WCP;         // waves across the columns
    static constexpr int NWR = kGuWaves / NWC;          // waves across the rows
    static constexpr int BM = 32 * WR * NWR;            // 128 rows (64 at three limbs)
    static constexpr int NA = L * BM / 32;              // A fragments per stage
    static constexpr int NB = 2 * kGuN / 32;            // 8 B fragments (4 gate, 4 up)
    static constexpr int NF = NA + NB;
    static constexpr int NL = 2 * NF;                   // wave-wide loads per stage
    static constexpr int LPW = (NL + kGuWaves - 1) / kGuWaves;
    static constexpr int STAGE = NF * kGuFrag;
};

// DN = false: gate/up, A = X digit planes (hm_dlay_x: [T][H/64][L][64])
// gathered by perm_tokens, out = gu [R x 2I] (tile: 128 gate + 128 up
// columns).  At L = 2 the A load units are whole 128-byte lines (a row's two
// planes of the stage), 8 rows a unit, stored at row r's 128 bytes with the
// 16-byte pieces rotated by (r / 2) % 8 (the paired fragment order, read
// conflict-free at gu_pair_read_offset); otherwise 16 rows of one plane's
// 64 bytes a unit (gu_frag_load_row/chunk).
// DN = true: down, A = Z digit planes (hm_dlay_z: [I/64][L][R][64]) of the
// grouped rows themselves (a 16-row load unit is one contiguous kilobyte),
// out = y [R x H] (tile: 256 down columns; the "gate" half of the gate/up
// tile is its first 128 columns, the "up" half the next).
template <int L, bool DN>
__global__ __launch_bounds__(kGuThreads) void ring_gemm_kernel(
    const int8_t* __restrict__ xdig, const float* __restrict__ xscale,
    const int32_t* __restrict__ xdsum, int tokens, int H, int I, int experts,
    const int8_t* __restrict__ packed, const float* __restrict__ scale,
    const int32_t* __restrict__ zp, const int32_t* __restrict__ counts,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ perm_tokens, int skinny,
    float* __restrict__ gu) {
    using T = GateUpTile<L>;
    // inner and output dimensions of the projection(s), output columns per
    // tile, the out row stride and the offset of the tile's second half
    const int K = DN ? I : H, N = DN ? H : I;
    constexpr int TN = DN ? 2 * kGuN : kGuN;
    const int64_t ldo = DN ? (int64_t)N : 2 * (int64_t)N;
    const int half = DN ? kGuN : N;
    constexpr int PG = DN ? 2 : 0, PU = DN ? 2 : 1;  // the halves' projections
    constexpr int BM = T::BM, NA = T::NA, NL = T::NL, LPW = T::LPW, WR = T::WR, WCP = T::WCP,
                  NWC = T::NWC, STAGE = T::STAGE;
    constexpr int RW = BM / HM_WAVE;  // waves that move one value per tile row
    constexpr int kS = kGuStages;
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
    const int E = experts;
    for (int e = tid; e < E; e += kGuThreads) {
        s_cnt[e] = counts[e];
        s_off[e] = offsets[e];
        s_sg[e] = scale[3 * e + PG];
        s_su[e] = scale[3 * e + PU];
        s_zg[e] = zp[3 * e + PG];
        s_zu[e] = zp[3 * e + PU];
    }
    __syncthreads();
    if (wave == 0) tile_prefix(s_cnt, E, BM, skinny, s_prefix);
    __syncthreads();
    const int nbn = N / TN;
    const TileRange tr = tile_range(s_prefix[E] * nbn);
    if (tr.ntiles == 0) return;
    const int nk = K / kGuKB;
    const int64_t tiles_k = hm_pad32(K) / 32;  // K tiles of one 32-column block

    auto info = [&](int i) __attribute__((always_inline)) {
        const int j = tr.jbeg + i * tr.step;
        const int gm = j / nbn;
        TileInfo t;
        t.e = locate_expert(s_prefix, E, gm);
        const int mt = gm - s_prefix[t.e];
        t.g0 = s_off[t.e] + mt * BM;
        t.nrows = min(BM, s_cnt[t.e] - mt * BM);
        t.n0 = (j % nbn) * TN;
        return t;
    };
    // A rows of the tile rows: their tokens (gate/up) or the grouped rows
    // themselves (down); rows past nrows repeat the last row
    auto fetch_rows = [&](const TileInfo& t, int m) __attribute__((always_inline)) {
        if (wave < RW) {
            const int r = HM_WAVE * wave + lane;
            if constexpr (DN) s_rt[m][r] = t.g0 + min(r, t.nrows - 1);
            else dma4(perm_tokens + t.g0 + min(r, t.nrows - 1), &s_rt[m][HM_WAVE * wave]);
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
    // this wave's load units: unit u = fragment u/2, half (K step) u%2.
    // Unit c of wave w is u = w + 8c; when the stage's NL units do not fill
    // every wave's LPW slots, the waves below NFULL issue LPW loads per stage
    // and the others LPW-1.
    constexpr int NFULL = NL - kGuWaves * (LPW - 1);
    static_assert(NFULL >= 1 && NFULL <= kGuWaves, "load units");
    const bool full = wave < NFULL;
    int dst[LPW];
#pragma unroll
    for (int c = 0; c < LPW; ++c) {
        const int u = (wave + kGuWaves * c) % NL;
        dst[c] = (u >> 1) * kGuFrag + 1024 * (u & 1);
    }
    // per-lane sources at stage 0 and their advance per stage (A: the next
    // 64-byte chunk of the digit layout; B: two 1 KB tiles)
    constexpr bool PAIRED = !DN && L == 2;
    const int astep = DN ? L * tokens * kGuKB : L * kGuKB;
    int sstep[LPW];
#pragma unroll
    for (int c = 0; c < LPW; ++c) sstep[c] = ((wave + kGuWaves * c) % NL) / 2 < NA ? astep : 2048;
    auto make_src = [&](const TileInfo& t, int m, const int8_t* (&src)[LPW]) {
        const int ch = gu_frag_load_chunk(lane);
#pragma unroll
        for (int c = 0; c < LPW; ++c) {
            const int u = (wave + kGuWaves * c) % NL;
            const int f = u >> 1, h = u & 1;
            if (f < NA) {
                if constexpr (PAIRED) {
                    // unit u: rows 8 (u % 4) .. +7 of 32-row block u / 4
                    const int r = 8 * (u & 3) + (lane >> 3);
                    const int tok = s_rt[m][32 * (u >> 2) + r];
                    src[c] = xdig + (int64_t)tok * (L * K) + 16 * ((lane & 7) ^ ((r >> 1) & 7));
                } else {
                    const int l = f / (BM / 32), i = f % (BM / 32);
                    const int tok = s_rt[m][32 * i + gu_frag_load_row(lane, h)];
                    src[c] = DN ? xdig + ((int64_t)l * tokens + tok) * kGuKB + 16 * ch
                                : xdig + (int64_t)tok * (L * K) + l * kGuKB + 16 * ch;
                }
            } else {
                const int fb = f - NA;
                const int64_t cb = t.n0 / 32 + (DN ? fb : (fb & 3));
                src[c] = packed + hm_proj_offset(t.e, DN ? 2 : fb >> 2, H, I) +
                         (cb * tiles_k + h) * 1024 + 16 * lane;
            }
        }
    };
    // load c of a stage exists on this wave
    auto has_unit = [&](int c) __attribute__((always_inline)) { return c < LPW - 1 || full; };
    auto issue = [&](int slot, const int8_t* const (&src)[LPW], int ks) {
        int8_t* st = ring + slot * STAGE;
#pragma unroll
        for (int c = 0; c < LPW; ++c)
            if (has_unit(c)) dma16(src[c] + (int64_t)ks * sstep[c], st + dst[c]);
    };
    // wait until at most n stages of this wave's loads are in flight
    auto vm_wait_stages = [&](auto nst) __attribute__((always_inline)) {
        constexpr int n = decltype(nst)::value;
        if (full) vm_wait<n * LPW>();
        else vm_wait<n * (LPW - 1)>();
    };

    int rd[2], rdp[2][2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        rd[h] = gu_frag_read_offset(lane, h);
#pragma unroll
        for (int l = 0; l < 2; ++l) rdp[h][l] = gu_pair_read_offset(lane, h, l);
    }
    v4i fa[2][WR][L], fb[2][2 * WCP];
    v16i acc[WR][L][2 * WCP];
    const int8_t* src[LPW];  // per-lane sources of this wave's loads

    // ---- the K loop.  Stream stage s (the tiles' stages back to back) lives
    // in ring slot s % kS.  Step s: wait until this wave's loads of stage s+1
    // have landed, workgroup barrier, refill the slot of stage s-1 with stage
    // s+kS-1, then the MFMAs of stage s (fragments in registers) while the
    // fragments of stage s+1 are read: register set h as soon as the last
    // MFMA of K step h that uses it has issued.  The slot refilled at step s
    // was read during step s-2, so the barrier needs only this wave's older
    // LDS reads complete: the reads of step s-1 stay in flight across it
    // (a barrier that drained them left all eight waves waiting on the
    // LDS together once per stage, the matrix pipes idle).
    constexpr int NJ = 2 * WCP;                 // B fragments per K step
    constexpr int NM = WR * L * NJ;             // MFMAs per K step
    constexpr int RPS = 2 * (WR * L + NJ);      // LDS fragment reads per step
    static_assert(RPS <= 15, "lgkmcnt range");
    auto read_a = [&](int slot, int h, int ii, int l) __attribute__((always_inline)) {
        if constexpr (PAIRED)
            fa[h][ii][l] = lds16(ring + slot * STAGE + (wr * WR + ii) * 2 * kGuFrag + rdp[h][l]);
        else
            fa[h][ii][l] = lds16(ring + slot * STAGE + (l * (BM / 32) + wr * WR + ii) * kGuFrag + rd[h]);
    };
    auto read_b = [&](int slot, int h, int j) __attribute__((always_inline)) {
        const int fbi = j < WCP ? wc * WCP + j : kGuN / 32 + wc * WCP + (j - WCP);
        fb[h][j] = lds16(ring + slot * STAGE + (NA + fbi) * kGuFrag + 1024 * h + 16 * lane);
    };
    // K step h of the current stage; rslot: slot of the stage whose set-h
    // fragments are read meanwhile (-1: none); (h = 0) the step's refill
    // loads into dslot from source stage dks go out after the first MFMAs.
    // The sched_barriers keep this order.
    auto kstep_h = [&](auto hc, auto first, int rslot, int dslot, int dks) __attribute__((always_inline)) {
        constexpr int h = decltype(hc)::value;
#pragma unroll
        for (int mi = 0; mi < NM; ++mi) {
            const int ii = mi / (L * NJ), l = (mi / NJ) % L, j = mi % NJ;
            if constexpr (decltype(first)::value)
                acc[ii][l][j] = mfma32(fa[h][ii][l], fb[h][j], v16i{});
            else
                acc[ii][l][j] = mfma32(fa[h][ii][l], fb[h][j], acc[ii][l][j]);
            if (h == 0 && mi < LPW && dslot >= 0 && has_unit(mi))
                dma16(src[mi] + (int64_t)dks * sstep[mi], ring + dslot * STAGE + dst[mi]);
            if (rslot >= 0) {
                if (j == NJ - 1) read_a(rslot, h, ii, l);
                if (ii == WR - 1 && l == L - 1) read_b(rslot, h, j);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (h == 0 && dslot >= 0)
#pragma unroll
            for (int c = NM; c < LPW; ++c)
                if (has_unit(c)) dma16(src[c] + (int64_t)dks * sstep[c], ring + dslot * STAGE + dst[c]);
    };
    auto read_all = [&](int slot) __attribute__((always_inline)) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int ii = 0; ii < WR; ++ii)
#pragma unroll
                for (int l = 0; l < L; ++l) read_a(slot, h, ii, l);
#pragma unroll
            for (int j = 0; j < NJ; ++j) read_b(slot, h, j);
        }
    };

    // ---- stream prologue: tile 0's rows, metadata and first kS-1 stages
    TileInfo cur = info(0);
    int m = 0;
    fetch_rows(cur, 0);
    vm_wait<0>();
    lds_barrier();
    fetch_row_meta(0);
    make_src(cur, 0, src);
    int slot0 = 0;  // ring slot of the current tile's stage 0
#pragma unroll
    for (int s = 0; s < kS - 1; ++s) issue(s, src, s);
    vm_wait_stages(std::integral_constant<int, kS - 2>{});
    lds_barrier();

    for (int i = 0; i < tr.ntiles; ++i) {
        const bool has_next = i + 1 < tr.ntiles;
        const int mn = m ^ 1;
        TileInfo nxt = cur;
        if (has_next) nxt = info(i + 1);
        // a wave whose rows all lie past the tile's last row (an expert's
        // partial last tile) skips its fragment reads and MFMAs
        const bool act = 32 * WR * wr < cur.nrows;
        // Step ks.  Phase A (ks <= nk-kS): refill with this tile's stage
        // ks+kS-1; phase B: with the next tile's stage ks+kS-1-nk.
        auto step = [&](int ks, auto first, auto phase_b, auto active) __attribute__((always_inline)) {
            constexpr bool B = decltype(phase_b)::value, ACT = decltype(active)::value;
            // stage ks+1 of the stream has landed once at most the stages
            // after it that are already issued (ks+2 .. ks+kS-2) are in flight
            if (!B || has_next) vm_wait_stages(std::integral_constant<int, kS - 3>{});
            else if (ks + 1 < nk) vm_wait<0>();
            if constexpr (ACT) lds_barrier_keep<RPS>();
            else lds_barrier();
            const int dslot = !B || has_next ? (slot0 + ks + kS - 1) % kS : -1;
            const int dks = B ? ks + kS - 1 - nk : ks + kS - 1;
            if (decltype(first)::value && has_next) fetch_rows(nxt, mn);
            if constexpr (ACT) {
                const int rslot = ks + 1 < nk ? (slot0 + ks + 1) % kS : -1;
                kstep_h(std::integral_constant<int, 0>{}, first, rslot, dslot, dks);
                kstep_h(std::integral_constant<int, 1>{}, std::false_type{}, rslot, -1, 0);
            } else if (dslot >= 0) {
                issue(dslot, src, dks);
            }
        };
        auto tile_k = [&](auto active) __attribute__((always_inline)) {
            // stage 0's fragments (landed and published by the previous
            // step's barrier)
            if constexpr (decltype(active)::value) read_all(slot0);
            step(0, std::true_type{}, std::false_type{}, active);
            int ks = 1;
#pragma clang loop unroll(disable)
            for (; ks <= nk - kS; ++ks) step(ks, std::false_type{}, std::false_type{}, active);
            if (has_next) {
                // the next tile's loads start now: their sources (its row
                // tokens have landed, a stage issued after them has) and its
                // row metadata
                if (nk < 2 * kS) {
                    vm_wait<0>();
                    lds_barrier();
                }
                make_src(nxt, mn, src);
                fetch_row_meta(mn);
            }
#pragma clang loop unroll(disable)
            for (; ks < nk; ++ks) step(ks, std::false_type{}, std::true_type{}, active);
        };
        if (act) tile_k(std::true_type{});
        else tile_k(std::false_type{});

        // ---- epilogue (the next tile's first kS-2 stages are in flight):
        // g and u into the row's two halves of gu.  The zero-point
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
                    const int rq = r0 + 8 * q + 4 * (lane >> 5);  // rows rq .. rq+3
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
                        float* grow = gu + (int64_t)(cur.g0 + rq + t4) * ldo + cur.n0 +
                                      32 * wc * WCP + (lane & 31);
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
                                if constexpr (DN) {
                                    grow[32 * j] = g;
                                    grow[half + 32 * j] = u;
                                } else {
                                    // g | u is read once, by the SwiGLU pass:
                                    // streamed, so that it does not evict the
                                    // operands the other tiles read again
                                    __builtin_nontemporal_store(g, &grow[32 * j]);
                                    __builtin_nontemporal_store(u, &grow[half + 32 * j]);
                                }
                            }
                        }
                    }
                }
            }
        };
        if (act) {
            if ((s_zg[cur.e] | s_zu[cur.e]) != 0) epilogue(std::true_type{});
            else epilogue(std::false_type{});
        }
        // next tile
        slot0 = (slot0 + nk) % kS;
        m = mn;
        cur = nxt;
    }
}

bool gateup_shape_ok(int64_t H, int64_t I, int64_t E, int32_t limbs) {
    // |P_l| <= H * 128 * 255 < 2^31 keeps every limb partial exact: H <= 65536
    return limbs >= 1 && limbs <= 3 && E >= 1 && E <= kMaxExperts && H <= 65536 &&
           I <= (1 << 20) && H % kGuKB == 0 && H / kGuKB >= kGuStages && I % kGuN == 0;
}

// The down projection on the ring kernel: K = I in 64-byte stages, N = H in
// 256-column tiles.
bool down_ring_ok(int64_t H, int64_t I, int64_t E, int32_t limbs) {
    return limbs >= 1 && limbs <= 3 && E >= 1 && E <= kMaxExperts && I <= 65536 &&
           H <= (1 << 20) && I % kGuKB == 0 && I / kGuKB >= kGuStages && H % (2 * kGuN) == 0;
}

// Down: skinny groups (split K, when asked for), then the tiles of the
// others on the ring kernel, or on limb_gemm_kernel where the ring's shape
// conditions do not hold.
template <int L>
int launch_down(const hm_layer* layer, const int8_t* zdig, const float* zscale,
                const int32_t* zdsum, int64_t R, const int32_t* counts, const int32_t* offsets,
                float* y, bool split_k, hipStream_t stream) {
    if (!down_ring_ok(layer->hidden, layer->intermediate, layer->experts, L))
        return launch_l<L>(layer, zdig, zscale, zdsum, R, counts, offsets, y, split_k, stream);
    const bool sk = split_k && skinny_ok(layer->intermediate, layer->hidden, L, false);
    if (sk) {
        const int rc = launch_skinny<L, false>(layer, zdig, zscale, zdsum, R, nullptr, counts,
                                               offsets, y, stream, false);
        if (rc) return rc;
    }
    hipLaunchKernelGGL((ring_gemm_kernel<L, true>), dim3((unsigned)persistent_grid()),
                       dim3(kGuThreads), 0, stream, zdig, zscale, zdsum, (int)R,
                       (int)layer->hidden, (int)layer->intermediate, (int)layer->experts,
                       static_cast<const int8_t*>(layer->packed), layer->scale,
                       layer->zero_point, counts, offsets, nullptr, sk ? kSkinnyRows : 0, y);
    HM_LAUNCHED();
    return HM_OK;
}

template <int L>
int launch_gateup(const hm_layer* layer, const int8_t* xdig, const float* xscale,
                  const int32_t* xdsum, int64_t tokens, const int32_t* counts,
                  const int32_t* offsets, const int32_t* perm_tokens, float* gu, bool split_k,
                  hipStream_t stream) {
    // skinny groups (split K, when asked for; its start opens an armed stage
    // timer), then the tiles of the others
    const bool sk = split_k && skinny_ok(layer->hidden, layer->intermediate, L, true);
    if (sk) {
        const int rc = launch_skinny<L, true>(layer, xdig, xscale, xdsum, tokens, perm_tokens,
                                              counts, offsets, gu, stream, true);
        if (rc) return rc;
    }
    HM_STAGE_LAUNCH(!sk, false, (ring_gemm_kernel<L, false>), dim3((unsigned)persistent_grid()),
                    dim3(kGuThreads), 0, stream, xdig, xscale, xdsum, (int)tokens,
                    (int)layer->hidden, (int)layer->intermediate, (int)layer->experts,
                    static_cast<const int8_t*>(layer->packed), layer->scale, layer->zero_point,
                    counts, offsets, perm_tokens, sk ? kSkinnyRows : 0, gu);
    HM_LAUNCHED();
    return HM_OK;
}

}  // namespace

// Shape preconditions of the MFMA kernels: K in 128-byte stages (enough of
// them for the stream's look-ahead, a count the B register ring divides),
// N in whole workgroup column blocks, E <= 256 (tables in LDS).
bool hm_mfma_gateup_ok(int64_t H, int64_t I, int64_t E, int32_t limbs) {
    return gateup_shape_ok(H, I, E, limbs);
}

bool hm_mfma_down_ok(int64_t H, int64_t I, int64_t E, int32_t limbs) {
    return down_ring_ok(H, I, E, limbs) || shape_ok(I, H, E, limbs);
}

// gu [R x 2I]: the gate and up values of every grouped row (X digits in the
// hm_dlay_x layout).  The first kernel of the gate/up stage (its start opens
// an armed stage timer).
int hm_launch_gateup_i8_mfma(const hm_layer* layer, int32_t limbs, const int8_t* xdig,
                             const float* xscale, const int32_t* xdsum, int64_t tokens,
                             const int32_t* counts, const int32_t* offsets,
                             const int32_t* perm_tokens, int64_t R, float* gu, bool split_k,
                             hipStream_t stream) {
    if (tokens > INT_MAX || R > INT_MAX) return HM_ERR_OVERFLOW;
    switch (limbs) {
    case 1: return launch_gateup<1>(layer, xdig, xscale, xdsum, tokens, counts, offsets, perm_tokens, gu, split_k, stream);
    case 2: return launch_gateup<2>(layer, xdig, xscale, xdsum, tokens, counts, offsets, perm_tokens, gu, split_k, stream);
    case 3: return launch_gateup<3>(layer, xdig, xscale, xdsum, tokens, counts, offsets, perm_tokens, gu, split_k, stream);
    default: return HM_ERR_INVALID;
    }
}

// y [R x H] from the Z digit planes (hm_dlay_z; one scale per row).
int hm_launch_down_i8_mfma(const hm_layer* layer, int32_t limbs, const int32_t* counts,
                           const int32_t* offsets, int64_t R, const int8_t* zdig,
                           const float* zscale, const int32_t* zdsum, float* y, bool split_k,
                           hipStream_t stream) {
    if (R > INT_MAX) return HM_ERR_OVERFLOW;
    switch (limbs) {
    case 1: return launch_down<1>(layer, zdig, zscale, zdsum, R, counts, offsets, y, split_k, stream);
    case 2: return launch_down<2>(layer, zdig, zscale, zdsum, R, counts, offsets, y, split_k, stream);
    case 3: return launch_down<3>(layer, zdig, zscale, zdsum, R, counts, offsets, y, split_k, stream);
    default: return HM_ERR_INVALID;
    }
}
