// Factorized radial-form probe: the per-edge work that the reference's
// factorized compact radial form adds before any channel contraction, measured
// at the shapes this evaluator runs.  That form splines the radial network's
// 64-wide last hidden layer (a 1 KiB coefficient row per edge) and projects it
// to the P x C path weights with the network's last linear layer
// (compact_radial.hpp:18-27; mace_kokkos_factorized_lifecycle.cpp:4126-4170);
// this evaluator instead splines the P x C path weights themselves (a
// 16 P C-byte row per edge, layers.hip).
//
//   radial_probe [edges N rows] ...
//
// Default cases: the medium workload (369,244 edges within r_cut, N = P C =
// 10 x 128), the same with one table per unordered element pair (Agnesi
// transform, 6 pairs of 256 intervals), and the wide water workload
// (1,610,342 edges, N = 17 x 256).  For each case:
//   1. spline: the 64 hidden units of every edge from its coefficient row
//      (64 cubics, row and local coordinate per edge drawn at random);
//   2. projection: the same, then the 64 x N product on the FP32 matrix cores
//      (v_mfma_f32_32x32x2f32; a wave holds the hidden units of 64 edges as
//      two 32-row blocks and streams the projection from L2 in the operand
//      layout, one float4 per lane per four MFMAs).  The N columns of each
//      edge are summed in the accumulators (the contraction with the features,
//      which the form would do next, is left out: the time is a lower bound
//      on the form's R1 forward) and checked against a double-precision host
//      sum on sampled edges.
// Each is timed with HIP events over 10 launches after 2 warmups; prints the
// time per launch and, for the projection, its FP32 rate (2 x 64 x N flops
// per edge) against the 157.3 TFLOP/s FP32 matrix peak.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

namespace {

#define CHECK(x)                                                                         \
    do {                                                                                 \
        hipError_t err_ = (x);                                                           \
        if (err_ != hipSuccess) {                                                        \
            std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(err_));               \
            std::exit(1);                                                                \
        }                                                                                \
    } while (0)

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kHidden = 64;        // hidden units splined per edge
constexpr int kWaveEdges = 64;     // edges per wave: two 32-row MFMA blocks
constexpr int kWaves = 4;          // waves per workgroup
constexpr double kPeakTflops = 157.3;

// Hidden units of the lane's edge in MFMA A-operand order: lane half hf holds
// unit 8c + 4hf + q as element q of float4 c (c = 0..7), the units that MFMA
// q of chunk c takes from that half (the two halves give the two k of one
// MFMA, so the 32 MFMAs of a chunk pass sum every unit once).
__device__ __forceinline__ void hidden_units(const float4* __restrict__ table, const int* __restrict__ rows,
                                             const float* __restrict__ xs, int E, int e, int hf, float4 (&h)[8])
{
    if (e >= E) {
#pragma unroll
        for (int c = 0; c < 8; ++c) h[c] = make_float4(0.f, 0.f, 0.f, 0.f);
        return;
    }
    const float4* row = table + static_cast<size_t>(rows[e]) * kHidden;
    const float x = xs[e];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 k = row[8 * c + 4 * hf + q];
            v[q] = fmaf(fmaf(fmaf(k.w, x, k.z), x, k.y), x, k.x);
        }
        h[c] = make_float4(v[0], v[1], v[2], v[3]);
    }
}

// 1. spline only: out[e] = sum of the edge's 64 hidden units
__global__ void __launch_bounds__(256) spline_kernel(const float4* __restrict__ table, const int* __restrict__ rows,
                                                      const float* __restrict__ xs, int E, float* __restrict__ out)
{
    const int lane = threadIdx.x & 63;
    const int tile = blockIdx.x * kWaves + (threadIdx.x >> 6);
    const int hf = lane >> 5;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const int e = tile * kWaveEdges + 32 * b + (lane & 31);
        float4 h[8];
        hidden_units(table, rows, xs, E, e, hf, h);
        float s = 0.f;
#pragma unroll
        for (int c = 0; c < 8; ++c) s += (h[c].x + h[c].y) + (h[c].z + h[c].w);
        s += __shfl_xor(s, 32);
        if (hf == 0 && e < E) out[e] = s;
    }
}

// 2. spline + projection: out[e] = sum_n sum_k h[e][k] W[k][n].  Wp holds W
// in B-operand order: Wp[(nb * 8 + c) * 64 + lane] = W[8c + 4hf + q][32 nb +
// (lane & 31)], q = 0..3, for column block nb.
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) projection_kernel(const float4* __restrict__ table,
                                                          const int* __restrict__ rows,
                                                          const float* __restrict__ xs, int E,
                                                          const float4* __restrict__ Wp, int col_blocks,
                                                          float* __restrict__ out)
{
    const int lane = threadIdx.x & 63;
    const int tile = blockIdx.x * kWaves + (threadIdx.x >> 6);
    const int hf = lane >> 5;
    float4 h[2][8];
#pragma unroll
    for (int b = 0; b < 2; ++b) hidden_units(table, rows, xs, E, tile * kWaveEdges + 32 * b + (lane & 31), hf, h[b]);
    floatx16 acc[2];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[b][v] = 0.0f;
    // the projection as a stream of float4 chunks (chunk nb * 8 + c feeds the
    // eight MFMAs of chunk c of column block nb) through a ring of 8: seven
    // chunks in flight while one is multiplied (past the end the last chunk
    // is loaded again, so every step issues one load and the waits stay exact)
    const int chunks = col_blocks * 8;
    float4 ring[8];
#pragma unroll
    for (int d = 0; d < 7; ++d) ring[d] = Wp[static_cast<size_t>(d) * 64 + lane];
    for (int j = 0; j < chunks; j += 8) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const int next = min(j + c + 7, chunks - 1);
            ring[(c + 7) % 8] = Wp[static_cast<size_t>(next) * 64 + lane];
            // keep the load here: the scheduler would otherwise sink each
            // load to just before its use
            __builtin_amdgcn_sched_barrier(0);
            const float4 w = ring[c];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(h[b][c].x, w.x, acc[b], 0, 0, 0);
                acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(h[b][c].y, w.y, acc[b], 0, 0, 0);
                acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(h[b][c].z, w.z, acc[b], 0, 0, 0);
                acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(h[b][c].w, w.w, acc[b], 0, 0, 0);
            }
        }
    }
    // accumulator v holds row 8 (v >> 2) + 4 hf + (v & 3), column lane & 31:
    // sum the 32 columns across the lanes of the half
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            float s = acc[b][v];
#pragma unroll
            for (int o = 1; o < 32; o <<= 1) s += __shfl_xor(s, o);
            const int e = tile * kWaveEdges + 32 * b + 8 * (v >> 2) + 4 * hf + (v & 3);
            if ((lane & 31) == 0 && e < E) out[e] = s;
        }
}

template <class Launch>
double time_ms(Launch launch)
{
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
    for (int i = 0; i < 2; ++i) launch();
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    CHECK(hipEventRecord(a, nullptr));
    for (int i = 0; i < 10; ++i) launch();
    CHECK(hipEventRecord(b, nullptr));
    CHECK(hipEventSynchronize(b));
    float ms = 0.f;
    CHECK(hipEventElapsedTime(&ms, a, b));
    CHECK(hipEventDestroy(a));
    CHECK(hipEventDestroy(b));
    return ms / 10.0;
}

struct Case {
    const char* name;
    int edges, N, rows;
};

void run_case(const Case& cs)
{
    const int E = cs.edges, N = cs.N, R = cs.rows;
    if (E <= 0 || R <= 0 || N <= 0 || N % 32 != 0) {
        std::fprintf(stderr, "case %s: edges and rows must be positive and N a positive multiple of 32\n", cs.name);
        std::exit(2);
    }
    std::mt19937 gen(11);
    std::uniform_real_distribution<float> u(-1.f, 1.f), u01(0.f, 1.f);
    std::uniform_int_distribution<int> ur(0, R - 1);
    std::vector<float> table(static_cast<size_t>(R) * kHidden * 4), W(static_cast<size_t>(kHidden) * N), xs(E);
    std::vector<int> rows(E);
    for (auto& v : table) v = u(gen);
    for (auto& v : W) v = 0.125f * u(gen);
    for (int e = 0; e < E; ++e) {
        rows[e] = ur(gen);
        xs[e] = u01(gen);
    }
    const int col_blocks = N / 32;
    std::vector<float> Wp(static_cast<size_t>(kHidden) * N);
    for (int nb = 0; nb < col_blocks; ++nb)
        for (int c = 0; c < 8; ++c)
            for (int l = 0; l < 64; ++l)
                for (int q = 0; q < 4; ++q)
                    Wp[((static_cast<size_t>(nb) * 8 + c) * 64 + l) * 4 + q] =
                        W[static_cast<size_t>(8 * c + 4 * (l >> 5) + q) * N + 32 * nb + (l & 31)];

    float4 *d_table = nullptr, *d_Wp = nullptr;
    int* d_rows = nullptr;
    float *d_xs = nullptr, *d_out = nullptr;
    CHECK(hipMalloc(&d_table, table.size() * sizeof(float)));
    CHECK(hipMalloc(&d_Wp, Wp.size() * sizeof(float)));
    CHECK(hipMalloc(&d_rows, rows.size() * sizeof(int)));
    CHECK(hipMalloc(&d_xs, xs.size() * sizeof(float)));
    CHECK(hipMalloc(&d_out, static_cast<size_t>(E) * sizeof(float)));
    CHECK(hipMemcpy(d_table, table.data(), table.size() * sizeof(float), hipMemcpyHostToDevice));
    CHECK(hipMemcpy(d_Wp, Wp.data(), Wp.size() * sizeof(float), hipMemcpyHostToDevice));
    CHECK(hipMemcpy(d_rows, rows.data(), rows.size() * sizeof(int), hipMemcpyHostToDevice));
    CHECK(hipMemcpy(d_xs, xs.data(), xs.size() * sizeof(float), hipMemcpyHostToDevice));

    const int tiles = (E + kWaveEdges - 1) / kWaveEdges;
    const int blocks = (tiles + kWaves - 1) / kWaves;
    const double t_spline =
        time_ms([&] { spline_kernel<<<blocks, 64 * kWaves>>>(d_table, d_rows, d_xs, E, d_out); });
    const double t_proj = time_ms(
        [&] { projection_kernel<<<blocks, 64 * kWaves>>>(d_table, d_rows, d_xs, E, d_Wp, col_blocks, d_out); });

    // check sampled edges of the projection against a double host sum
    std::vector<float> out(E);
    CHECK(hipMemcpy(out.data(), d_out, out.size() * sizeof(float), hipMemcpyDeviceToHost));
    std::vector<double> wsum(kHidden, 0.0), wabs(kHidden, 0.0);
    for (int k = 0; k < kHidden; ++k)
        for (int n = 0; n < N; ++n) {
            wsum[k] += W[static_cast<size_t>(k) * N + n];
            wabs[k] += std::fabs(W[static_cast<size_t>(k) * N + n]);
        }
    double worst = 0.0;
    int checked = 0;
    for (int e = 0; e < E; e += 997) {
        double want = 0.0, scale = 0.0;
        for (int k = 0; k < kHidden; ++k) {
            const float* c = &table[(static_cast<size_t>(rows[e]) * kHidden + k) * 4];
            const double x = xs[e];
            const double h = ((static_cast<double>(c[3]) * x + c[2]) * x + c[1]) * x + c[0];
            want += h * wsum[k];
            scale += std::fabs(h) * wabs[k];
        }
        worst = std::max(worst, std::fabs(out[e] - want) / scale);
        ++checked;
    }
    const double flops = 2.0 * kHidden * N * static_cast<double>(E);
    const double tflops = flops / (t_proj * 1e-3) / 1e12;
    std::printf("%s: %d edges, N = %d, %d rows | spline %.4f ms | spline + projection %.4f ms = %.1f TFLOP/s "
                "(%.2f of %.1f) | %d edges checked, max error %.2e of sum |h||W|\n",
                cs.name, E, N, R, t_spline, t_proj, tflops, tflops / kPeakTflops, kPeakTflops, checked, worst);
    std::fflush(stdout);
    CHECK(hipFree(d_table));
    CHECK(hipFree(d_Wp));
    CHECK(hipFree(d_rows));
    CHECK(hipFree(d_xs));
    CHECK(hipFree(d_out));
    if (!(worst < 1e-5)) {
        std::fprintf(stderr, "%s: projection check failed\n", cs.name);
        std::exit(1);
    }
}

}  // namespace

int main(int argc, char** argv)
{
    std::vector<Case> cases;
    if (argc > 1) {
        if ((argc - 1) % 3 != 0) {
            std::fprintf(stderr, "usage: radial_probe [edges N rows] ...\n");
            return 2;
        }
        for (int i = 1; i + 2 < argc; i += 3)
            cases.push_back({"case", std::atoi(argv[i]), std::atoi(argv[i + 1]), std::atoi(argv[i + 2])});
    } else {
        cases = {{"medium (shared table)", 369244, 10 * 128, 256},
                 {"medium (per-pair tables)", 369244, 10 * 128, 6 * 256},
                 {"wide (water)", 1610342, 17 * 256, 256}};
    }
    for (const Case& c : cases) run_case(c);
    return 0;
}
