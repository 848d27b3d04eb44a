// gfx950 FP32 MFMA GEMMs of the node linears: H1 = M0 H1_W, A1 = Phi1 A1_W
// and their adjoints (reference mace.cpp:1690-1724, 2304-2340, 1664-1688,
// 2380-2458; the reference calls CBLAS / Kokkos batched GEMM for these), plus
// the pre_linear_up scalar x = M0_scalar P0 (+ residual) and its adjoint
// M0_adj += direct P0^T (mace_kokkos_h1_phi1.cpp:253-345, 511-553), which use
// the optional per-type bias and the accumulating store.
//
// All irrep blocks of one stage run in one launch (a group of up to
// kMaxGemmGroup GEMMs, tiles numbered consecutively across the group).  A
// 256-thread workgroup computes a 64 x 128 output tile with four waves of
// v_mfma_f32_32x32x2f32 (each wave 32 x 64: two 32 x 32 blocks), or, in
// launches too small to fill the chip, a 16 x 128 tile with four waves of
// v_mfma_f32_16x16x4f32 (each wave 16 x 32).  K is staged through LDS in
// slices of 16 (64-row tiles) or 32 (16-row tiles), the next slice's global
// loads in flight while the current one is multiplied.  Both operands are
// stored K-contiguous (the weight matrix is passed transposed, Bt[n][k]) so
// one ds_read_b128 feeds four MFMAs: lane group h supplies k = 8c + 4h + q
// (32 x 32 blocks, two groups) or k = 16c + 4h + q (16 x 16 blocks, four
// groups) to MFMA q of chunk c, the same k for both operands, which sums
// every k of the chunk exactly once.
#include <hip/hip_runtime.h>

#include "kernels.hpp"

namespace sxl {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kBN = 128, kPad = 4;
constexpr int kKMultiple = 32;  // K must be a multiple of every slice length

// 64-row tiles: four waves as 2 x 2, each 32 x 64 (two MFMA blocks), K
// staged in slices of 16: 15 KB of LDS and 78 VGPRs, six workgroups per CU
// where slices of 32 (27 KB, 96 VGPRs) allowed five and slices of 64 three.
// (Launches too small to fill the chip take the 16-row kernel below; a
// 32-row form of this kernel, four waves of one 32 x 32 block each, ran
// slower than the 16-row one at every size measured.)
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(6, 6))) gemm_group_kernel(GemmGroup grp)
{
    constexpr int kBM = 64;
    constexpr int kWN = 2;                       // waves along N
    constexpr int kNB = kBN / kWN / 32;          // 32 x 32 MFMA blocks per wave along N
    constexpr int kBK = 16;                      // K slice
    static_assert(kKMultiple % kBK == 0, "slice length divides the K multiple");
    __shared__ float As[kBM][kBK + kPad];
    __shared__ float Bs[kBN][kBK + kPad];
    const int b = blockIdx.x;
    int item = 0;
    while (item + 1 < grp.count && b >= grp.tile_start[item + 1]) ++item;
    const GemmArgs& g = grp.g[item];
    const int M = g.nodes * g.rows_per_node;
    const int K = g.K, N = g.Ncols;
    const int local = b - grp.tile_start[item];
    const int tiles_m = (M + kBM - 1) / kBM;
    const int row0 = (local % tiles_m) * kBM;
    const int col0 = (local / tiles_m) * kBN;
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int wm = wave / kWN, wn = wave % kWN;

    // global -> register staging: kBK / 4 threads per row (one float4 each),
    // kRowsPerPass rows per pass; A takes kAPasses passes, Bt kBPasses
    constexpr int kThreadsPerRow = kBK / 4, kRowsPerPass = 256 / kThreadsPerRow;
    constexpr int kAPasses = kBM / kRowsPerPass, kBPasses = kBN / kRowsPerPass;
    const int lr = t / kThreadsPerRow, lk = (t % kThreadsPerRow) * 4;
    const float* arow[kAPasses];
#pragma unroll
    for (int j = 0; j < kAPasses; ++j) {
        const int r = row0 + lr + kRowsPerPass * j;
        arow[j] = nullptr;
        if (r < M) {
            const int node = r / g.rows_per_node;
            const int m = r - node * g.rows_per_node;
            const long long gn = g.node_ids ? g.node_ids[node] : node;
            arow[j] = g.a.ptr + gn * g.a.node_stride + m * g.a.row_stride + lk;
        }
    }
    const float* brow[kBPasses];
#pragma unroll
    for (int j = 0; j < kBPasses; ++j) {
        const int n = col0 + lr + kRowsPerPass * j;
        brow[j] = n < N ? g.Bt + static_cast<size_t>(n) * K + lk : nullptr;
    }
    float4 ra[kAPasses], rb[kBPasses];
    auto fetch = [&](int k0) {
#pragma unroll
        for (int j = 0; j < kAPasses; ++j)
            ra[j] = arow[j] ? *reinterpret_cast<const float4*>(arow[j] + k0) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int j = 0; j < kBPasses; ++j)
            rb[j] = brow[j] ? *reinterpret_cast<const float4*>(brow[j] + k0) : make_float4(0.f, 0.f, 0.f, 0.f);
    };

    floatx16 acc[kNB];
#pragma unroll
    for (int j = 0; j < kNB; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[j][v] = 0.0f;

    fetch(0);
    const int arow_l = wm * 32 + (lane & 31);
    const int kh = 4 * (lane >> 5);
    for (int k0 = 0; k0 < K; k0 += kBK) {
#pragma unroll
        for (int j = 0; j < kAPasses; ++j) *reinterpret_cast<float4*>(&As[lr + kRowsPerPass * j][lk]) = ra[j];
#pragma unroll
        for (int j = 0; j < kBPasses; ++j) *reinterpret_cast<float4*>(&Bs[lr + kRowsPerPass * j][lk]) = rb[j];
        __syncthreads();
        if (k0 + kBK < K) fetch(k0 + kBK);
#pragma unroll
        for (int c = 0; c < kBK; c += 8) {
            const float4 a4 = *reinterpret_cast<const float4*>(&As[arow_l][c + kh]);
#pragma unroll
            for (int j = 0; j < kNB; ++j) {
                const float4 b4 = *reinterpret_cast<const float4*>(&Bs[wn * (kBN / kWN) + j * 32 + (lane & 31)][c + kh]);
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a4.x, b4.x, acc[j], 0, 0, 0);
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a4.y, b4.y, acc[j], 0, 0, 0);
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a4.z, b4.z, acc[j], 0, 0, 0);
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a4.w, b4.w, acc[j], 0, 0, 0);
            }
        }
        __syncthreads();
    }
    // accumulator v of block j holds row 8 (v >> 2) + 4 (lane >> 5) + (v & 3),
    // column j * 32 + (lane & 31): four runs of four consecutive rows, whose
    // (node, row in node) is found once per run and then stepped
    const int rpn = g.rows_per_node;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        int row = row0 + wm * 32 + 8 * q + 4 * (lane >> 5);
        int node = row / rpn;
        int m = row - node * rpn;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (row < M) {
                const long long gn = g.node_ids ? g.node_ids[node] : node;
                const long long base = gn * g.c.node_stride + m * g.c.row_stride;
#pragma unroll
                for (int j = 0; j < kNB; ++j) {
                    const int col = col0 + wn * (kBN / kWN) + j * 32 + (lane & 31);
                    if (col >= N) continue;
                    float value = acc[j][4 * q + u];
                    if (g.bias.ptr)
                        value += g.bias.ptr[g.bias.node_types[g.bias.node_base + node] * g.bias.type_stride +
                                            m * g.bias.row_stride + col];
                    float* dst = g.c.ptr + base + col;
                    if (g.accumulate) value += *dst;
                    *dst = value;
                }
            }
            ++row;
            if (++m == rpn) {
                m = 0;
                ++node;
            }
        }
    }
}

typedef float floatx4 __attribute__((ext_vector_type(4)));

// 16-row tiles for launches that leave most SIMDs idle even with 32-row
// tiles (small graphs), where each wave's chain of MFMAs sets the time: four
// waves side by side, each 16 x 32 (two blocks of v_mfma_f32_16x16x4f32:
// half the MFMA chain of a 32-row tile's wave), twice the workgroups, K
// staged through LDS in slices of 32.  Lane group h = lane >> 4 supplies
// k = c + 4h + q to MFMA q of chunk c (16 k), the same k for both operands,
// so one ds_read_b128 per operand feeds four MFMAs and every k of the chunk
// is summed exactly once.
__global__ void __launch_bounds__(256) gemm_group16_kernel(GemmGroup grp)
{
    constexpr int kBM = 16, kBK = 32, kWN = 4;
    constexpr int kNB = kBN / kWN / 16;  // 16 x 16 blocks per wave along N
    __shared__ float As[kBM][kBK + kPad];
    __shared__ float Bs[kBN][kBK + kPad];
    const int b = blockIdx.x;
    int item = 0;
    while (item + 1 < grp.count && b >= grp.tile_start[item + 1]) ++item;
    const GemmArgs& g = grp.g[item];
    const int M = g.nodes * g.rows_per_node;
    const int K = g.K, N = g.Ncols;
    const int local = b - grp.tile_start[item];
    const int tiles_m = (M + kBM - 1) / kBM;
    const int row0 = (local % tiles_m) * kBM;
    const int col0 = (local / tiles_m) * kBN;
    const int t = threadIdx.x;
    const int lane = t & 63, wn = t >> 6;

    // global -> register staging: 8 threads per row (one float4 each), 32
    // rows per pass: A (16 rows) by the first 128 threads, Bt in 4 passes
    constexpr int kThreadsPerRow = kBK / 4, kRowsPerPass = 256 / kThreadsPerRow;
    constexpr int kBPasses = kBN / kRowsPerPass;
    const int lr = t / kThreadsPerRow, lk = (t % kThreadsPerRow) * 4;
    const float* arow = nullptr;
    if (lr < kBM && row0 + lr < M) {
        const int r = row0 + lr;
        const int node = r / g.rows_per_node;
        const int m = r - node * g.rows_per_node;
        const long long gn = g.node_ids ? g.node_ids[node] : node;
        arow = g.a.ptr + gn * g.a.node_stride + m * g.a.row_stride + lk;
    }
    const float* brow[kBPasses];
#pragma unroll
    for (int j = 0; j < kBPasses; ++j) {
        const int n = col0 + lr + kRowsPerPass * j;
        brow[j] = n < N ? g.Bt + static_cast<size_t>(n) * K + lk : nullptr;
    }
    float4 ra, rb[kBPasses];
    auto fetch = [&](int k0) {
        ra = arow ? *reinterpret_cast<const float4*>(arow + k0) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int j = 0; j < kBPasses; ++j)
            rb[j] = brow[j] ? *reinterpret_cast<const float4*>(brow[j] + k0) : make_float4(0.f, 0.f, 0.f, 0.f);
    };

    floatx4 acc[kNB];
#pragma unroll
    for (int j = 0; j < kNB; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[j][v] = 0.0f;

    fetch(0);
    const int kq = 4 * (lane >> 4);
    for (int k0 = 0; k0 < K; k0 += kBK) {
        if (lr < kBM) *reinterpret_cast<float4*>(&As[lr][lk]) = ra;
#pragma unroll
        for (int j = 0; j < kBPasses; ++j) *reinterpret_cast<float4*>(&Bs[lr + kRowsPerPass * j][lk]) = rb[j];
        __syncthreads();
        if (k0 + kBK < K) fetch(k0 + kBK);
#pragma unroll
        for (int c = 0; c < kBK; c += 16) {
            const float4 a4 = *reinterpret_cast<const float4*>(&As[lane & 15][c + kq]);
#pragma unroll
            for (int j = 0; j < kNB; ++j) {
                const float4 b4 = *reinterpret_cast<const float4*>(&Bs[wn * 32 + j * 16 + (lane & 15)][c + kq]);
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.x, b4.x, acc[j], 0, 0, 0);
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.y, b4.y, acc[j], 0, 0, 0);
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.z, b4.z, acc[j], 0, 0, 0);
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.w, b4.w, acc[j], 0, 0, 0);
            }
        }
        __syncthreads();
    }
    // accumulator v of block j holds row 4 (lane >> 4) + v, column
    // j * 16 + (lane & 15): one run of four consecutive rows
    const int rpn = g.rows_per_node;
    int row = row0 + 4 * (lane >> 4);
    int node = row / rpn;
    int m = row - node * rpn;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        if (row < M) {
            const long long gn = g.node_ids ? g.node_ids[node] : node;
            const long long base = gn * g.c.node_stride + m * g.c.row_stride;
#pragma unroll
            for (int j = 0; j < kNB; ++j) {
                const int col = col0 + wn * 32 + j * 16 + (lane & 15);
                if (col >= N) continue;
                float value = acc[j][u];
                if (g.bias.ptr)
                    value += g.bias.ptr[g.bias.node_types[g.bias.node_base + node] * g.bias.type_stride +
                                        m * g.bias.row_stride + col];
                float* dst = g.c.ptr + base + col;
                if (g.accumulate) value += *dst;
                *dst = value;
            }
        }
        ++row;
        if (++m == rpn) {
            m = 0;
            ++node;
        }
    }
}

}  // namespace

hipError_t launch_gemm_group(GemmGroup grp, hipStream_t stream)
{
    if (grp.count < 0 || grp.count > kMaxGemmGroup) return hipErrorInvalidValue;
    int kept = 0;
    for (int i = 0; i < grp.count; ++i) {
        const GemmArgs& g = grp.g[i];
        const long long M = static_cast<long long>(g.nodes) * g.rows_per_node;
        if (M <= 0 || g.Ncols <= 0 || g.K <= 0) continue;
        if (g.K % kKMultiple != 0 || M > 0x7fffffff) return hipErrorInvalidValue;
        // float4 loads: row strides and bases must keep 16-byte alignment
        if (g.a.node_stride % 4 != 0 || g.a.row_stride % 4 != 0 ||
            reinterpret_cast<std::uintptr_t>(g.a.ptr) % 16 != 0 || reinterpret_cast<std::uintptr_t>(g.Bt) % 16 != 0)
            return hipErrorInvalidValue;
        grp.g[kept++] = g;
    }
    grp.count = kept;
    auto number_tiles = [&](int bm) {
        int tiles = 0;
        for (int i = 0; i < kept; ++i) {
            const long long M = static_cast<long long>(grp.g[i].nodes) * grp.g[i].rows_per_node;
            grp.tile_start[i] = tiles;
            tiles += static_cast<int>(((M + bm - 1) / bm) * ((grp.g[i].Ncols + kBN - 1) / kBN));
        }
        grp.tile_start[kept] = tiles;
        return tiles;
    };
    // 64-row tiles unless they leave most compute units with at most one
    // workgroup (256 CUs, five or six resident per CU); then 16-row tiles
    // (medium shape, per call, against 32-row tiles: 135 atoms 247 -> 232 us,
    // 625 atoms 396 -> 388-392 us, 2,560 and 5,000 atoms unchanged)
    int tiles = number_tiles(64);
    if (tiles == 0) return hipSuccess;
    if (tiles < 2 * 256) {
        tiles = number_tiles(16);
        gemm_group16_kernel<<<tiles, 256, 0, stream>>>(grp), note_launch();
    } else {
        gemm_group_kernel<<<tiles, 256, 0, stream>>>(grp), note_launch();
    }
    return hipGetLastError();
}

}  // namespace sxl
