// hm_gemm_f32_mfma.hip -- grouped FP32-weight expert GEMMs on the FP32
// matrix cores (v_mfma_f32_32x32x2_f32) for gfx950: the A5' path
// (ExpertExecutor.cpp:97-131 on CpuTensorBackend::matmul, :87-131).
//
// The reference sums each output sequentially in FP32; here the K terms are
// summed by the matrix cores in an order of their own, so the results are
// within the FP32 path's 1e-3 of the reference, not bit-identical (the same
// contract as the FMA tiles in hm_gemm.hip, which remain for other shapes).
//
// Workgroup: 4 waves, tile BM = 64 grouped rows x 128 weight rows (gate/up:
// 64 gate + the same 64 up columns; down: 128 output columns).  Wave (wr,
// wc) owns rows 32*wr .. +31 and two 32-column MFMA accumulators (gate/up:
// the gate and the up block of columns 32*wc; down: columns 64*wc and
// 64*wc + 32).  K moves in stages of 32 floats through a 3-slot LDS ring
// filled by 16-byte direct loads (global_load_lds).  Lane (g, i) =
// (lane/32, lane%32) supplies A = x[row i][k] and B = W[col i][k]; with a
// float4 of each per lane, MFMA step j of a group of four takes
// k = 8q + 4g + j, so every lane reads 16 contiguous bytes per four MFMAs.
// Rows of a stage are 128 bytes; the 16-byte chunk c of row r is stored at
// slot c ^ (r % 8), which spreads a reader's 32 rows over the LDS banks.
#include "hm_device.h"
#include "hm_lds_dma.h"

#include <limits.h>

namespace {

constexpr int kFThreads = 256;
constexpr int kFBM = 64;            // grouped rows per tile
constexpr int kFBN = 128;           // weight rows per tile
constexpr int kFBK = 32;            // K floats per stage
constexpr int kFSlots = 3;
constexpr int kFRow = kFBK * 4;     // bytes per staged row
constexpr int kFStage = (kFBM + kFBN) * kFRow;  // 24 KB

typedef float v16f __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v16f mfma_f32(float a, float b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// GATEUP: z[g, n] = silu(x_g . Wg[n]) * (x_g . Wu[n]), x_g = hidden[perm[g]],
// n in [0, I); tile columns n0 .. n0+63.  DOWN: y[g, n] = z_g . Wd[n],
// n in [0, H); tile columns n0 .. n0+127.
template <bool GATEUP>
__global__ __launch_bounds__(kFThreads) void expert_f32_mfma_kernel(
    const float* __restrict__ x, int K, int N, int experts, const float* __restrict__ packed,
    int hidden, int inter, const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ perm_tokens, float* __restrict__ out) {
    __shared__ __attribute__((aligned(1024))) char ring[kFSlots][kFStage];
    __shared__ int s_src[kFBM];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = wave >> 1, wc = wave & 1;
    int64_t e64, mt;
    if (!hm_locate_tile(counts, experts, kFBM, blockIdx.x, &e64, &mt)) return;
    const int e = (int)e64;
    const int64_t g0 = offsets[e] + mt * kFBM;
    const int rows = (int)min((int64_t)kFBM, (int64_t)counts[e] - mt * kFBM);
    const int64_t n0 = (int64_t)blockIdx.y * (GATEUP ? kFBN / 2 : kFBN);
    if (tid < kFBM) {
        const int r = tid < rows ? tid : rows - 1;  // rows past the group repeat its last
        s_src[tid] = GATEUP ? perm_tokens[g0 + r] : (int)(g0 + r);
    }
    __syncthreads();
    // this wave's DMA rows: activation rows 16*wave .. +15 (2 loads), weight
    // rows 32*wave .. +31 (4 loads); lane l covers row base + l/8, slot l%8
    const int slot = lane & 7, rsub = lane >> 3;
    const float* asrc[2];
    for (int i = 0; i < 2; ++i) {
        const int r = 16 * wave + 8 * i + rsub;
        const int c = slot ^ (r & 7);
        asrc[i] = x + (int64_t)s_src[r] * K + 4 * c;
    }
    const float* wbase = packed + (int64_t)e * 3 * hidden * inter;
    const float* wsrc[4];
    for (int i = 0; i < 4; ++i) {
        const int r = 32 * wave + 8 * i + rsub;  // 0 .. 127
        const int c = slot ^ (r & 7);
        int64_t row;
        const float* proj;
        if (GATEUP) {
            proj = wbase + (int64_t)(r >= 64 ? 1 : 0) * hidden * inter;
            row = n0 + (r & 63);
        } else {
            proj = wbase + 2 * (int64_t)hidden * inter;
            row = n0 + r;
        }
        wsrc[i] = proj + row * K + 4 * c;
    }
    const int nk = K / kFBK;
    auto issue = [&](int sl, int ks) {
        char* st = ring[sl];
        const int64_t k0 = (int64_t)ks * kFBK;
        for (int i = 0; i < 2; ++i) dma16(asrc[i] + k0, st + (16 * wave + 8 * i) * kFRow);
        for (int i = 0; i < 4; ++i)
            dma16(wsrc[i] + k0, st + kFBM * kFRow + (32 * wave + 8 * i) * kFRow);
    };
    v16f acc0 = {}, acc1 = {};
    const int g = lane >> 5, li = lane & 31;
    // this lane's rows in the stage: activation row 32*wr + li; weight rows
    // (gate/up) 32*wc + li and 64 + 32*wc + li, (down) 64*wc + li, +32
    const int ar = 32 * wr + li;
    const int br0 = GATEUP ? 32 * wc + li : 64 * wc + li;
    const int br1 = GATEUP ? 64 + 32 * wc + li : 64 * wc + 32 + li;
    issue(0, 0);
    if (nk > 1) issue(1, 1);
    for (int ks = 0; ks < nk; ++ks) {
        if (ks + 1 < nk) wait_vmcnt<6>();
        else wait_vmcnt<0>();
        lds_barrier();  // stage ks landed for every wave; stage ks-1 fully read
        if (ks + 2 < nk) issue((ks + 2) % kFSlots, ks + 2);
        const char* st = ring[ks % kFSlots];
        const char* arow = st + ar * kFRow;
        const char* b0row = st + kFBM * kFRow + br0 * kFRow;
        const char* b1row = st + kFBM * kFRow + br1 * kFRow;
#pragma unroll
        for (int q = 0; q < kFBK / 8; ++q) {
            const int c = 2 * q + g;  // 16-byte chunk of k = 8q + 4g .. +3
            const float4 a = *reinterpret_cast<const float4*>(arow + 16 * (c ^ (ar & 7)));
            const float4 b0 = *reinterpret_cast<const float4*>(b0row + 16 * (c ^ (br0 & 7)));
            const float4 b1 = *reinterpret_cast<const float4*>(b1row + 16 * (c ^ (br1 & 7)));
            acc0 = mfma_f32(a.x, b0.x, acc0);
            acc1 = mfma_f32(a.x, b1.x, acc1);
            acc0 = mfma_f32(a.y, b0.y, acc0);
            acc1 = mfma_f32(a.y, b1.y, acc1);
            acc0 = mfma_f32(a.z, b0.z, acc0);
            acc1 = mfma_f32(a.z, b1.z, acc1);
            acc0 = mfma_f32(a.w, b0.w, acc0);
            acc1 = mfma_f32(a.w, b1.w, acc1);
        }
    }
    // D[r][c]: r = 8*(v/4) + 4*g + v%4, c = lane%32
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int r = 32 * wr + 8 * (v >> 2) + 4 * g + (v & 3);
        if (r >= rows) continue;
        float* orow = out + (g0 + r) * (int64_t)N;
        if (GATEUP) {
            orow[n0 + 32 * wc + li] = __fmul_rn(hm_silu(acc0[v]), acc1[v]);
        } else {
            orow[n0 + 64 * wc + li] = acc0[v];
            orow[n0 + 64 * wc + 32 + li] = acc1[v];
        }
    }
}

}  // namespace

// Shapes the FP32 MFMA kernels take (16-byte aligned operands).
bool hm_f32_mfma_gateup_ok(int64_t H, int64_t I) {
    return H % kFBK == 0 && I % (kFBN / 2) == 0 && H <= INT_MAX / 4 && I <= INT_MAX / 4;
}
bool hm_f32_mfma_down_ok(int64_t H, int64_t I) {
    return I % kFBK == 0 && H % kFBN == 0 && H <= INT_MAX / 4 && I <= INT_MAX / 4;
}

int hm_launch_gateup_f32_mfma(const hm_layer* L, const float* hidden, const int32_t* counts,
                              const int32_t* offsets, const int32_t* perm_tokens, int64_t R,
                              int64_t max_tiles, float* z, hipStream_t stream) {
    if (R > INT_MAX || max_tiles > INT_MAX) return HM_ERR_OVERFLOW;
    const dim3 grid((unsigned)max_tiles, (unsigned)(L->intermediate / (kFBN / 2)));
    HM_STAGE_LAUNCH(true, true, expert_f32_mfma_kernel<true>, grid, dim3(kFThreads), 0, stream,
                    hidden, (int)L->hidden, (int)L->intermediate, (int)L->experts,
                    static_cast<const float*>(L->packed), (int)L->hidden, (int)L->intermediate,
                    counts, offsets, perm_tokens, z);
    HM_LAUNCHED();
    return HM_OK;
}

int hm_launch_down_f32_mfma(const hm_layer* L, const float* z, const int32_t* counts,
                            const int32_t* offsets, int64_t R, int64_t max_tiles, float* y,
                            hipStream_t stream) {
    if (R > INT_MAX || max_tiles > INT_MAX) return HM_ERR_OVERFLOW;
    const dim3 grid((unsigned)max_tiles, (unsigned)(L->hidden / kFBN));
    hipLaunchKernelGGL(expert_f32_mfma_kernel<false>, grid, dim3(kFThreads), 0, stream, z,
                       (int)L->intermediate, (int)L->hidden, (int)L->experts,
                       static_cast<const float*>(L->packed), (int)L->hidden,
                       (int)L->intermediate, counts, offsets, nullptr, y);
    HM_LAUNCHED();
    return HM_OK;
}
