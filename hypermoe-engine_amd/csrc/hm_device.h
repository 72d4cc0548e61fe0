// hm_device.h -- device helpers shared by the gfx950 kernels.
//
// Wave64 reductions, the device restatement of glibc 2.35 expf, and the
// integer-limb fixed-point split used by the INT8 expert GEMMs.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>

#include "hm_moe.h"

#define HM_WAVE 64

// Error plumbing shared by all launchers (defined in hm_runtime.hip).
void hm_record_hip_error(hipError_t e);
#define HM_HIP(expr)                                   \
    do {                                               \
        hipError_t hm_e_ = (expr);                     \
        if (hm_e_ != hipSuccess) {                     \
            hm_record_hip_error(hm_e_);                \
            return HM_ERR_RUNTIME;                     \
        }                                              \
    } while (0)
#define HM_LAUNCHED() HM_HIP(hipGetLastError())
#define HM_REQUIRE(cond) \
    do { if (!(cond)) return HM_ERR_INVALID; } while (0)

static inline hipStream_t hm_stream(void* s) { return static_cast<hipStream_t>(s); }

// Stage timing.  While a block call times a stage, `start` and `stop` hold
// two events: the stage's first kernel is launched with hipExtLaunchKernelGGL
// taking `start` at its own start, the last one `stop` at its own end, so
// the pair brackets the stage's kernels and none of the gaps around them
// (hipEventRecord between launches adds a marker packet and its gap).  Both
// are null otherwise and HM_STAGE_LAUNCH is an ordinary launch.  Per host
// thread (hm_runtime.hip), like the reference's single-caller backends.
struct hm_stage_timer {
    hipEvent_t start;
    hipEvent_t stop;
};
hm_stage_timer& hm_timer();
#define HM_STAGE_LAUNCH(first, last, kernel, grid, block, lds, stream, ...)                  \
    hipExtLaunchKernelGGL(kernel, grid, block, lds, stream,                                 \
                          (first) ? hm_timer().start : nullptr,                             \
                          (last) ? hm_timer().stop : nullptr, 0, __VA_ARGS__)

// A decode step (T <= 16) fuses the grouping into the router's select
// kernel; its last workgroup is found with a device counter that the
// step's first kernel zeroes.
struct hm_decode_fusion {
    int32_t* counters;   // [0]: the select's completion counter
    int n_counters;
    int32_t* counts;
    int32_t* offsets;
    int32_t* perm_tokens;
    float* perm_weights;
    int32_t* slots;
};

// RMSNorm folded into the decode router's first kernel: the rows it reads
// are the layer input h, normalised with gamma and eps on the fly; x_out
// [T x H] receives RMSNorm(h), the rows every later kernel of the block
// reads.  force_seq: every row takes the reference's sequential sum of
// squares (the certified interval is skipped).  gamma == nullptr: no norm.
struct hm_norm_fold {
    const float* gamma;
    float* x_out;
    float eps;
    int force_seq;
};

// ---------------------------------------------------------------------------
// Wave64 reductions (all 64 lanes must be active).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float hm_wave_max_f32(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, HM_WAVE));
    return v;
}

__device__ __forceinline__ double hm_wave_sum_f64(double v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, HM_WAVE);
    return v;
}

__device__ __forceinline__ int hm_wave_sum_i32(int v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, HM_WAVE);
    return v;
}

__device__ __forceinline__ unsigned long long hm_wave_max_u64(unsigned long long v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        unsigned long long o = __shfl_xor(v, m, HM_WAVE);
        v = o > v ? o : v;
    }
    return v;
}

// Max / sum over each 16-lane row of the wave with DPP (quad_perm 1032,
// quad_perm 2301, row_half_mirror, row_mirror): every lane of the row gets
// the result.  Max and integer sums are order-free, so the result is exact.
__device__ __forceinline__ float hm_dpp_f32(float v, int ctrl_sel) {
    const int x = __builtin_bit_cast(int, v);
    int y;
    switch (ctrl_sel) {
    case 0: y = __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false); break;
    case 1: y = __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false); break;
    case 2: y = __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false); break;
    default: y = __builtin_amdgcn_update_dpp(0, x, 0x140, 0xF, 0xF, false); break;
    }
    return __builtin_bit_cast(float, y);
}
__device__ __forceinline__ float hm_row16_max(float v) {
#pragma unroll
    for (int c = 0; c < 4; ++c) v = fmaxf(v, hm_dpp_f32(v, c));
    return v;
}
__device__ __forceinline__ int hm_row16_sum(int v) {
#pragma unroll
    for (int c = 0; c < 4; ++c) v += __builtin_bit_cast(int, hm_dpp_f32(__builtin_bit_cast(float, v), c));
    return v;
}

// Whole-wave max / integer sum without LDS: DPP within each 16-lane row,
// then the four row results through v_readlane (uniform result).
__device__ __forceinline__ float hm_wave_max_dpp(float v) {
    const float r = hm_row16_max(v);
    const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, r), 0));
    const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, r), 16));
    const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, r), 32));
    const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, r), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}
__device__ __forceinline__ int hm_wave_sum_dpp(int v) {
    const int r = hm_row16_sum(v);
    return __builtin_amdgcn_readlane(r, 0) + __builtin_amdgcn_readlane(r, 16) +
           __builtin_amdgcn_readlane(r, 32) + __builtin_amdgcn_readlane(r, 48);
}

// The same for 64-bit values (both halves through the same DPP pattern).
__device__ __forceinline__ unsigned long long hm_dpp_u64(unsigned long long v, int ctrl_sel) {
    const float lo = hm_dpp_f32(__builtin_bit_cast(float, (unsigned)(v & 0xffffffffull)), ctrl_sel);
    const float hi = hm_dpp_f32(__builtin_bit_cast(float, (unsigned)(v >> 32)), ctrl_sel);
    return ((unsigned long long)__builtin_bit_cast(unsigned, hi) << 32) | __builtin_bit_cast(unsigned, lo);
}
__device__ __forceinline__ unsigned long long hm_readlane_u64(unsigned long long v, int l) {
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(v & 0xffffffffull), l);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(v >> 32), l);
    return ((unsigned long long)hi << 32) | lo;
}
__device__ __forceinline__ unsigned long long hm_wave_max_u64_dpp(unsigned long long v) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const unsigned long long o = hm_dpp_u64(v, c);
        v = o > v ? o : v;
    }
    unsigned long long m = hm_readlane_u64(v, 0);
#pragma unroll
    for (int r = 16; r < HM_WAVE; r += 16) {
        const unsigned long long o = hm_readlane_u64(v, r);
        m = o > m ? o : m;
    }
    return m;
}
// The same maximum kept in the vector unit to the end: after the row
// steps, row_bcast:15 hands rows 0 and 2 on to rows 1 and 3 and
// row_bcast:31 row 1 on to rows 2 and 3 (rows outside the row mask keep
// their own value), so lane 63 holds the wave's maximum.
__device__ __forceinline__ unsigned long long hm_wave_max_u64_bcast(unsigned long long v) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const unsigned long long o = hm_dpp_u64(v, c);
        v = o > v ? o : v;
    }
    {
        const int lo = (int)(unsigned)(v & 0xffffffffull), hi = (int)(unsigned)(v >> 32);
        const unsigned olo = (unsigned)__builtin_amdgcn_update_dpp(lo, lo, 0x142, 0xa, 0xf, false);
        const unsigned ohi = (unsigned)__builtin_amdgcn_update_dpp(hi, hi, 0x142, 0xa, 0xf, false);
        const unsigned long long o = ((unsigned long long)ohi << 32) | olo;
        v = o > v ? o : v;
    }
    {
        const int lo = (int)(unsigned)(v & 0xffffffffull), hi = (int)(unsigned)(v >> 32);
        const unsigned olo = (unsigned)__builtin_amdgcn_update_dpp(lo, lo, 0x143, 0xc, 0xf, false);
        const unsigned ohi = (unsigned)__builtin_amdgcn_update_dpp(hi, hi, 0x143, 0xc, 0xf, false);
        const unsigned long long o = ((unsigned long long)ohi << 32) | olo;
        v = o > v ? o : v;
    }
    return hm_readlane_u64(v, HM_WAVE - 1);
}
// Sum of doubles over the wave (row DPP, then the four rows in ascending
// row order); callers use it only where any summation order gives the
// same result.
__device__ __forceinline__ double hm_wave_sum_f64_dpp(double v) {
#pragma unroll
    for (int c = 0; c < 4; ++c)
        v += __builtin_bit_cast(double, hm_dpp_u64(__builtin_bit_cast(unsigned long long, v), c));
    double s = __builtin_bit_cast(double, hm_readlane_u64(__builtin_bit_cast(unsigned long long, v), 0));
#pragma unroll
    for (int r = 16; r < HM_WAVE; r += 16)
        s += __builtin_bit_cast(double, hm_readlane_u64(__builtin_bit_cast(unsigned long long, v), r));
    return s;
}

// glibc 2.35 expf restated for host and device (hm_expf.h); matches the host
// libm expf on every float input (exhaustive check, tests/test_expf_parity.py).
#include "hm_expf.h"

// A 16-byte load that the caches stream past (a value read once: the
// nontemporal hint keeps it from displacing operands that are read again).
__device__ __forceinline__ float4 hm_load_stream(const float4* p) {
    typedef float hm_v4f __attribute__((ext_vector_type(4)));
    const hm_v4f v = __builtin_nontemporal_load(reinterpret_cast<const hm_v4f*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

// SiLU exactly as src/tensor/activation/Activation.cpp:44 computes it:
// value / (1 + expf(-value)) in float.
__device__ __forceinline__ float hm_silu(float v) {
    return __fdiv_rn(v, __fadd_rn(1.0f, hm_expf(-v)));
}
// The same with the expf table in LDS (hm_load_exp2_table).
__device__ __forceinline__ float hm_silu_t(float v, const unsigned long long* table) {
    return __fdiv_rn(v, __fadd_rn(1.0f, hm_expf_t(-v, table)));
}
// hm_silu_t for |v| < 88 (hm_expf_small_t).
__device__ __forceinline__ float hm_silu_small_t(float v, const unsigned long long* table) {
    return __fdiv_rn(v, __fadd_rn(1.0f, hm_expf_small_t(-v, table)));
}
// Copies the expf table into a 32-entry LDS array (threads 0..31 write; the
// caller synchronises before use).
__device__ __forceinline__ void hm_load_exp2_table(unsigned long long* lds_table) {
    if (threadIdx.x < 32) lds_table[threadIdx.x] = kHmExp2Table[threadIdx.x];
}

// ---------------------------------------------------------------------------
// Integer-limb fixed point (build-owned numeric format).
//   range(L) = 127 * (256^L - 1) / 255
//   inv = range / amax, s = amax / range (float divisions)
//   n   = clamp(rint(x * inv), -range, range)
//   n   = sum_l d_l 256^l with balanced digits d_l in [-128, 127]
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ int hm_limb_range(int limbs) {
    return limbs == 1 ? 127 : limbs == 2 ? 32639 : 8355711;
}

__device__ __forceinline__ int hm_fixed_point(float x, float inv, float range) {
    float v = rintf(__fmul_rn(x, inv));
    v = fminf(fmaxf(v, -range), range);
    return (int)v;
}

// Digit l of n (l = 0 least significant).
__device__ __forceinline__ int hm_digit(int n, int l) {
    int d = 0;
    for (int i = 0; i <= l; ++i) {
        d = ((n + 128) & 255) - 128;
        n = (n - d) / 256;
    }
    return d;
}

// All L digits of n (|n| <= range(L)): the same digits as hm_digit, with
// shifts (n - d is a multiple of 256, so >> 8 divides exactly); the top
// digit is what remains, already in [-128, 127].
template <int L>
__device__ __forceinline__ void hm_digits(int n, int (&d)[L]) {
#pragma unroll
    for (int l = 0; l < L - 1; ++l) {
        d[l] = ((n + 128) & 255) - 128;
        n = (n - d[l]) >> 8;
    }
    d[L - 1] = n;
}

// c = (float)P_{L-1}; c = fmaf(c, 256, (float)P_l) for l = L-2 .. 0.
__device__ __forceinline__ float hm_recombine(const int* p, int limbs) {
    float c = (float)p[limbs - 1];
    for (int l = limbs - 2; l >= 0; --l) c = __builtin_fmaf(c, 256.0f, (float)p[l]);
    return c;
}

// Digit-plane layouts.  Digit (plane l, row r, k) of a block of digit rows
// sits at r * row + l * plane + (k >> 6) * chunk + (k & 63): K is cut into
// 64-byte chunks (the ring GEMMs' K stage), K64 = K rounded up to 64.
//   planes  [L][rows][K]          the op-level layout (hm_limb_quantize_rows)
//   X       [T][K64/64][L][64]    token rows: a row's L planes of one chunk
//                                 are L * 64 contiguous bytes (one 128-byte
//                                 line at L = 2), read gathered by token
//   Z       [K64/64][L][R][64]    grouped rows: one plane's chunk of
//                                 consecutive rows is contiguous (a 16-row
//                                 load unit is one kilobyte)
// Pad digits (K <= k < K64) are never read.
struct hm_dlay {
    int64_t row, plane, chunk;
};
__host__ __device__ __forceinline__ int64_t hm_pad64(int64_t v) { return (v + 63) & ~(int64_t)63; }
__host__ __device__ __forceinline__ hm_dlay hm_dlay_planes(int64_t rows, int64_t K) {
    return hm_dlay{K, rows * K, 64};
}
__host__ __device__ __forceinline__ hm_dlay hm_dlay_x(int L, int64_t K) {
    return hm_dlay{L * hm_pad64(K), 64, 64 * (int64_t)L};
}
__host__ __device__ __forceinline__ hm_dlay hm_dlay_z(int L, int64_t rows) {
    return hm_dlay{64, 64 * rows, 64 * rows * (int64_t)L};
}
__host__ __device__ __forceinline__ int64_t hm_dlay_off(const hm_dlay& d, int l, int64_t r,
                                                        int64_t k) {
    return r * d.row + l * d.plane + (k >> 6) * d.chunk + (k & 63);
}

// One wave quantises one FP32 row of n = 256*nv floats to L fixed-point
// digit planes: the row max gives the step (inv = range / max|x|), every
// element becomes rint(x * inv) split into L digits.  The row is in
// registers, lane: floats 4*(lane + 64 i) .. +3 in v[i].  Digit (l, k) of
// the row goes to digits + l * plane + (k >> 6) * chunk + (k & 63) (lay's
// plane and chunk strides, digits at the row's start; 4 bytes per lane and
// float4), its digit sum to dsum[l * dsum_stride] (when dsum is set), the
// scale max|x| / range to *scale.  Shared by the row-quantisation kernels
// and the routers' select kernels, so all of them write the same bytes.
constexpr int kHmQuantMaxV = 16;  // n <= 4096
template <int L>
__device__ __forceinline__ void hm_quantize_row_values(const float4* v, int nv,
                                                       int8_t* __restrict__ digits,
                                                       const hm_dlay& lay, float* scale,
                                                       int32_t* __restrict__ dsum,
                                                       int64_t dsum_stride) {
    const int lane = threadIdx.x & (HM_WAVE - 1);
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < kHmQuantMaxV; ++i) {
        if (i < nv)
            amax = fmaxf(fmaxf(amax, fmaxf(fabsf(v[i].x), fabsf(v[i].y))),
                         fmaxf(fabsf(v[i].z), fabsf(v[i].w)));
    }
    amax = hm_wave_max_dpp(amax);
    const float range = (float)hm_limb_range(L);
    const float inv = amax > 0.0f ? __fdiv_rn(range, amax) : 0.0f;
    int dl[L];
#pragma unroll
    for (int l = 0; l < L; ++l) dl[l] = 0;
#pragma unroll
    for (int i = 0; i < kHmQuantMaxV; ++i) {
        if (i < nv) {
            int d0[L], d1[L], d2[L], d3[L];
            hm_digits<L>(hm_fixed_point(v[i].x, inv, range), d0);
            hm_digits<L>(hm_fixed_point(v[i].y, inv, range), d1);
            hm_digits<L>(hm_fixed_point(v[i].z, inv, range), d2);
            hm_digits<L>(hm_fixed_point(v[i].w, inv, range), d3);
#pragma unroll
            for (int l = 0; l < L; ++l) {
                const uint32_t word = (uint32_t)(d0[l] & 255) | ((uint32_t)(d1[l] & 255) << 8) |
                                      ((uint32_t)(d2[l] & 255) << 16) | ((uint32_t)(d3[l] & 255) << 24);
                const int64_t k = 4 * (int64_t)(lane + HM_WAVE * i);
                *reinterpret_cast<uint32_t*>(digits + hm_dlay_off(lay, l, 0, k)) = word;
                dl[l] += d0[l] + d1[l] + d2[l] + d3[l];
            }
        }
    }
#pragma unroll
    for (int l = 0; l < L; ++l) {
        const int sm = hm_wave_sum_dpp(dl[l]);
        if (lane == 0 && dsum) dsum[(int64_t)l * dsum_stride] = sm;
    }
    if (lane == 0) *scale = amax > 0.0f ? __fdiv_rn(amax, range) : 0.0f;
}

// The same, reading the row (16-byte aligned) from memory.
template <int L>
__device__ __forceinline__ void hm_quantize_row_wave(const float* __restrict__ xrow, int nv,
                                                     int8_t* __restrict__ digits,
                                                     const hm_dlay& lay, float* scale,
                                                     int32_t* __restrict__ dsum,
                                                     int64_t dsum_stride) {
    const int lane = threadIdx.x & (HM_WAVE - 1);
    const float4* xr = reinterpret_cast<const float4*>(xrow);
    float4 v[kHmQuantMaxV];
#pragma unroll
    for (int i = 0; i < kHmQuantMaxV; ++i)
        if (i < nv) v[i] = xr[lane + HM_WAVE * i];
    hm_quantize_row_values<L>(v, nv, digits, lay, scale, dsum, dsum_stride);
}

// Where a fused row quantisation writes (digits == nullptr: none).
struct hm_row_quant {
    int8_t* digits;    // the X layout (hm_dlay_x): [rows][n64 / 64][limbs][64]
    float* scales;     // [rows]
    int32_t* dsum;     // [limbs][rows] or nullptr
    int32_t limbs;
};

// Grouped-GEMM tile lookup: tiles of expert e are ceil(counts[e]/tile_m),
// experts in ascending id.  Which expert, and which tile of it, does linear
// tile index `tile` name?  False when `tile` is past the last tile.
__device__ __forceinline__ bool hm_locate_tile(const int32_t* __restrict__ counts,
                                               int64_t experts, int tile_m, int64_t tile,
                                               int64_t* expert_out, int64_t* tile_in_expert) {
    // Wave-parallel: 64 experts at a time, an inclusive scan of their tile
    // counts, a ballot for the first expert whose tiles reach past `tile`.
    // Every lane of the wave must be active.
    const int lane = threadIdx.x & (HM_WAVE - 1);
    int64_t base = 0;  // tiles of the experts before this chunk
    for (int64_t c0 = 0; c0 < experts; c0 += HM_WAVE) {
        const int64_t e = c0 + lane;
        const int64_t n = e < experts ? ((int64_t)counts[e] + tile_m - 1) / tile_m : 0;
        int64_t incl = n;
#pragma unroll
        for (int sft = 1; sft < HM_WAVE; sft <<= 1) {
            const int64_t o = __shfl_up(incl, sft, HM_WAVE);
            if (lane >= sft) incl += o;
        }
        const int64_t total = __shfl(incl, HM_WAVE - 1, HM_WAVE);
        if (tile < base + total) {
            const unsigned long long m = __ballot(base + incl > tile);
            const int first = __ffsll((long long)m) - 1;
            const int64_t before = __shfl(incl - n, first, HM_WAVE);
            *expert_out = c0 + first;
            *tile_in_expert = tile - base - before;
            return true;
        }
        base += total;
    }
    return false;
}

// ---------------------------------------------------------------------------
// INT8 expert weight layout on the device ("tiles"; hm_pack_layer).
// A projection W [N x K] (N output columns, K inner: gate/up N = I, K = H;
// down N = H, K = I) is zero-padded to N32 x K32 (multiples of 32) and cut
// into 32 x 32 tiles; tile (cb, kb) is 1024 contiguous bytes at
// (cb * K32/32 + kb) * 1024, and inside it the 16 bytes of lane l are
// W[32 cb + l % 32][32 kb + 16 (l / 32) .. +15] at 16 l.  One wave-wide
// 16-byte load of a tile is therefore the B operand of
// v_mfma_i32_32x32x32_i8 for columns 32 cb .. +31 and K step kb, read as one
// contiguous kilobyte.  Every projection takes H32 * I32 bytes; projection p
// of expert e starts at (3 e + p) * H32 * I32.
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ int64_t hm_pad32(int64_t v) { return (v + 31) & ~(int64_t)31; }
__host__ __device__ __forceinline__ int64_t hm_tile_offset(int64_t n, int64_t k, int64_t K32) {
    return ((n >> 5) * (K32 >> 5) + (k >> 5)) * 1024 + ((n & 31) + 32 * ((k >> 4) & 1)) * 16 +
           (k & 15);
}
__host__ __device__ __forceinline__ int64_t hm_proj_bytes(int64_t H, int64_t I) {
    return hm_pad32(H) * hm_pad32(I);
}
// Start of projection p (0 gate, 1 up, 2 down) of expert e.
__host__ __device__ __forceinline__ int64_t hm_proj_offset(int64_t e, int p, int64_t H, int64_t I) {
    return (3 * e + p) * hm_proj_bytes(H, I);
}

// Float total order key for top-k: larger score first, equal scores (with
// -0 == +0) broken by the lower expert id; 0 is never a valid key.
__device__ __forceinline__ unsigned long long hm_rank_key(float v, unsigned int id) {
    unsigned int u = v == 0.0f ? 0u : __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (0xffffffffu - id);
}
