// Ahead-of-time R1 HIP plugin for one model contract (the reference's
// symmetrix_jit_hip_plugin_query_v1 artifact, jit_hip_plugin_abi.h:226-269):
// the second-interaction tensor product over the reference's packets, with
// its radial spline layout and caller-provided harmonics.
//
//   forward  (receiver owner, jit_codegen.py:884-1016): output[i][lme][k] =
//            sum over active edges of receiver i of sum_t cg_t R_p(t)(r)[k]
//            Y[lm1_t] H[src][lm2_t][k]
//   source   (source owner, jit_codegen.py:1018-1110): source_adjoint[s][lm2][k]
//            += sum over active edges from s of sum_t cg_t R_p(t)(r)[k]
//            Y[lm1_t] A[recv][lme_t][k], compensated (Kahan) sums
//   edge     (edge owner, jit_codegen.py:1314-1424): directed_forces[e] -=
//            sum_k sum_t cg_t H[src][lm2_t][k] A[recv][lme_t][k]
//            (R'_p Y[lm1_t] r_hat + R_p grad Y[lm1_t])
//
// The term pattern is the compiled R1Shape of the contract's harmonic orders
// (r1_shapes.inc) and the coefficients are the contract's, compiled in
// (r1_plugin_<contract>.inc, from gen_r1_plugin.py).  Launch shapes for
// gfx950: one workgroup of `channels` threads per receiver (forward) or
// source (reverse feature adjoint), one wave per edge with the lanes over
// channels (forces), grid-stride loops over at most the caller's persistent
// block count.  The evaluation point is formed in FP32 from the FP64 length,
// as the reference's FP32 plugins do.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstddef>
#include <cstdint>

#include "../../include/symmetrix_amd_r1_plugin.h"
#include "device_math.hpp"
#include "r1_shapes.inc"
#include SXL_R1_PLUGIN_INC

namespace {

using Shape = R1Shape<SXL_R1_PLUGIN_EDGE_LMAX, SXL_R1_PLUGIN_SOURCE_LMAX>;
constexpr int C = sxl_r1_plugin::kChannels;
constexpr int NLM1 = (SXL_R1_PLUGIN_EDGE_LMAX + 1) * (SXL_R1_PLUGIN_EDGE_LMAX + 1);
constexpr int NLM2 = (SXL_R1_PLUGIN_SOURCE_LMAX + 1) * (SXL_R1_PLUGIN_SOURCE_LMAX + 1);
constexpr int NLME = Shape::NLME;
constexpr int NP = Shape::NP;
constexpr int NT = Shape::NT;
static_assert(NT == sxl_r1_plugin::kTerms, "the contract's terms are the compiled shape's");
static_assert(C % 64 == 0 && C <= 256, "channels per workgroup: whole waves, at most 256");

constexpr int kForwardThreads = C;
constexpr int kSourceThreads = C;
constexpr int kEdgeThreads = 256;  // four edges per workgroup, one per wave
constexpr int kPersistentBlocksPerCU = 8;

__device__ __forceinline__ int pair_type(int left, int right, int count)
{
    return left <= right ? left * (2 * count - left - 1) / 2 + right : right * (2 * count - right - 1) / 2 + left;
}

struct Point {
    int interval;
    float x, xx, xxx;
};

// evaluation point in FP32 from the FP64 length, clamped to the grid
__device__ __forceinline__ Point evaluation_point(const SymmetrixJitHipRadialSplineV1& s, double radius)
{
    const float r = static_cast<float>(radius), x0 = static_cast<float>(s.x0), h = static_cast<float>(s.h);
    int iv = static_cast<int>(floorf((r - x0) / h));
    float x = r - x0 - h * static_cast<float>(iv);
    if (iv < 0) {
        iv = 0;
        x = 0.0f;
    } else if (iv >= static_cast<int>(s.intervals)) {
        iv = static_cast<int>(s.intervals) - 1;
        x = h;
    }
    return {iv, x, x * x, x * x * x};
}

// the four coefficients of function `fn` at the point's interval
__device__ __forceinline__ void coefficients(const SymmetrixJitHipRadialSplineV1& s, int edge_type, int interval,
                                             int fn, float c[4])
{
    const float* base = static_cast<const float*>(s.coefficients) +
                        (static_cast<size_t>(edge_type) * s.intervals + interval) * 4 * s.functions + fn;
#pragma unroll
    for (int q = 0; q < 4; ++q) c[q] = base[static_cast<size_t>(q) * s.functions];
}

__global__ void __launch_bounds__(kForwardThreads) forward_kernel(SymmetrixJitHipR1ForwardArgsV1 a)
{
    const int k = threadIdx.x;
    const float* Yall = static_cast<const float*>(a.harmonics_values);
    const float* H = static_cast<const float*>(a.neighbor_features);
    float* out = static_cast<float*>(a.output);
    const int na = static_cast<int>(a.active_type_count);
    for (int64_t i = blockIdx.x; i < a.num_nodes; i += gridDim.x) {
        float value[NLME];
#pragma unroll
        for (int q = 0; q < NLME; ++q) value[q] = 0.0f;
        const int rt = a.type_to_active[a.node_types[i]];
        const int e0 = a.first_neigh[i], e1 = e0 + a.num_neigh[i];
        for (int e = e0; e < e1; ++e) {
            const double radius = a.radius[e];
            if (!(radius < a.cutoff)) continue;
            const int src = a.neigh_indices[e];
            const int et = pair_type(rt, a.type_to_active[a.neigh_types[e]], na);
            const Point pt = evaluation_point(a.radial, radius);
            float R[NP];
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                float c[4];
                coefficients(a.radial, et, pt.interval, p * C + k, c);
                R[p] = c[0] + c[1] * pt.x + c[2] * pt.xx + c[3] * pt.xxx;
            }
            float Y[NLM1], Hs[NLM2];
#pragma unroll
            for (int q = 0; q < NLM1; ++q) Y[q] = Yall[static_cast<size_t>(e) * NLM1 + q];
#pragma unroll
            for (int q = 0; q < NLM2; ++q) Hs[q] = H[(static_cast<size_t>(src) * NLM2 + q) * C + k];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const float product = R[Shape::term_p[t]] * Y[Shape::term_lm1[t]] * Hs[Shape::term_lm2[t]];
                value[Shape::term_lme[t]] += static_cast<float>(sxl_r1_plugin::kCoefficients[t]) * product;
            }
        }
        float* o = out + static_cast<size_t>(i) * NLME * C;
#pragma unroll
        for (int q = 0; q < NLME; ++q) o[q * C + k] = value[q];
    }
}

__global__ void __launch_bounds__(kSourceThreads) source_kernel(SymmetrixJitHipR1SourceArgsV1 a)
{
    const int k = threadIdx.x;
    const float* Yall = static_cast<const float*>(a.harmonics_values);
    const float* A = static_cast<const float*>(a.output_adjoint);
    float* out = static_cast<float*>(a.source_adjoint);
    const int na = static_cast<int>(a.active_type_count);
    for (int64_t s = blockIdx.x; s < a.num_nodes; s += gridDim.x) {
        float value[NLM2], comp[NLM2];
#pragma unroll
        for (int q = 0; q < NLM2; ++q) value[q] = comp[q] = 0.0f;
        for (int t0 = a.source_offsets[s]; t0 < a.source_offsets[s + 1]; ++t0) {
            const int e = a.source_edges[t0];
            const double radius = a.radius[e];
            if (!(radius < a.cutoff)) continue;
            const int recv = a.edge_receivers[e];
            const int et = pair_type(a.type_to_active[a.node_types[recv]], a.type_to_active[a.neigh_types[e]], na);
            const Point pt = evaluation_point(a.radial, radius);
            float R[NP];
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                float c[4];
                coefficients(a.radial, et, pt.interval, p * C + k, c);
                R[p] = c[0] + c[1] * pt.x + c[2] * pt.xx + c[3] * pt.xxx;
            }
            float Y[NLM1], Ar[NLME];
#pragma unroll
            for (int q = 0; q < NLM1; ++q) Y[q] = Yall[static_cast<size_t>(e) * NLM1 + q];
#pragma unroll
            for (int q = 0; q < NLME; ++q) Ar[q] = A[(static_cast<size_t>(recv) * NLME + q) * C + k];
            // per (path, lm1, lm2) row: its terms' coefficients against the
            // receiver's adjoint, times R Y, into the source's lm2 sum
            float row = 0.0f;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                row += static_cast<float>(sxl_r1_plugin::kCoefficients[t]) * Ar[Shape::term_lme[t]];
                if (t + 1 == NT || Shape::term_tr[t + 1] != Shape::term_tr[t]) {
                    const int lm2 = Shape::term_lm2[t];
                    const float contribution = R[Shape::term_p[t]] * Y[Shape::term_lm1[t]] * row;
                    const float corrected = contribution - comp[lm2];
                    const float updated = value[lm2] + corrected;
                    comp[lm2] = (updated - value[lm2]) - corrected;
                    value[lm2] = updated;
                    row = 0.0f;
                }
            }
        }
        float* o = out + static_cast<size_t>(s) * NLM2 * C;
#pragma unroll
        for (int q = 0; q < NLM2; ++q) o[q * C + k] += value[q];
    }
}

__global__ void __launch_bounds__(kEdgeThreads) edge_kernel(SymmetrixJitHipR1EdgeArgsV1 a)
{
    const int lane = threadIdx.x & 63;
    const int64_t waves = static_cast<int64_t>(gridDim.x) * (kEdgeThreads / 64);
    const float* Yall = static_cast<const float*>(a.harmonics_values);
    const float* G = static_cast<const float*>(a.harmonics_gradients);
    const float* H = static_cast<const float*>(a.neighbor_features);
    const float* A = static_cast<const float*>(a.output_adjoint);
    const int na = static_cast<int>(a.active_type_count);
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * (kEdgeThreads / 64) + (threadIdx.x >> 6); e < a.num_edges;
         e += waves) {
        const double radius = a.radius[e];
        if (!(radius < a.cutoff)) continue;  // whole wave
        const int recv = a.edge_receivers[e], src = a.neigh_indices[e];
        const int et = pair_type(a.type_to_active[a.node_types[recv]], a.type_to_active[a.neigh_types[e]], na);
        const Point pt = evaluation_point(a.radial, radius);
        double xyz[3];
        float u[3];
        if (a.coordinates_are_unit) {
            for (int c = 0; c < 3; ++c)
                u[c] = a.coordinate_scalar_size == sizeof(float)
                           ? static_cast<const float*>(a.xyz)[3 * e + c]
                           : static_cast<float>(static_cast<const double*>(a.xyz)[3 * e + c]);
            for (int c = 0; c < 3; ++c) xyz[c] = static_cast<double>(u[c]) * radius;
        } else {
            for (int c = 0; c < 3; ++c) {
                xyz[c] = static_cast<const double*>(a.xyz)[3 * e + c];
                u[c] = static_cast<float>(xyz[c] / radius);
            }
        }
        float Y[NLM1], gx[NLM1], gy[NLM1], gz[NLM1];
        if (G) {
#pragma unroll
            for (int q = 0; q < NLM1; ++q) {
                gx[q] = G[(3 * static_cast<size_t>(e) + 0) * NLM1 + q];
                gy[q] = G[(3 * static_cast<size_t>(e) + 1) * NLM1 + q];
                gz[q] = G[(3 * static_cast<size_t>(e) + 2) * NLM1 + q];
            }
        } else {
            float unused[NLM1], dir[3];
            sxl::edge_harmonics<SXL_R1_PLUGIN_EDGE_LMAX, true>(xyz, radius, unused, gx, gy, gz, dir);
        }
#pragma unroll
        for (int q = 0; q < NLM1; ++q) Y[q] = Yall[static_cast<size_t>(e) * NLM1 + q];
        float f[3] = {0.0f, 0.0f, 0.0f};
        for (int k = lane; k < C; k += 64) {
            float R[NP], dR[NP];
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                float c[4];
                coefficients(a.radial, et, pt.interval, p * C + k, c);
                R[p] = c[0] + c[1] * pt.x + c[2] * pt.xx + c[3] * pt.xxx;
                dR[p] = c[1] + c[2] * (2.0f * pt.x) + c[3] * (3.0f * pt.xx);
            }
            float Hs[NLM2], Ar[NLME];
#pragma unroll
            for (int q = 0; q < NLM2; ++q) Hs[q] = H[(static_cast<size_t>(src) * NLM2 + q) * C + k];
#pragma unroll
            for (int q = 0; q < NLME; ++q) Ar[q] = A[(static_cast<size_t>(recv) * NLME + q) * C + k];
            float row = 0.0f;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                row += static_cast<float>(sxl_r1_plugin::kCoefficients[t]) * Ar[Shape::term_lme[t]];
                if (t + 1 == NT || Shape::term_tr[t + 1] != Shape::term_tr[t]) {
                    const int p = Shape::term_p[t], lm1 = Shape::term_lm1[t];
                    const float weighted = Hs[Shape::term_lm2[t]] * row;
                    const float radial_force = dR[p] * weighted * Y[lm1];
                    const float angular = R[p] * weighted;
                    f[0] += radial_force * u[0] + angular * gx[lm1];
                    f[1] += radial_force * u[1] + angular * gy[lm1];
                    f[2] += radial_force * u[2] + angular * gz[lm1];
                    row = 0.0f;
                }
            }
        }
        double fd[3];
        for (int c = 0; c < 3; ++c) {
            fd[c] = static_cast<double>(f[c]);
            for (int off = 32; off > 0; off >>= 1) fd[c] += __shfl_xor(fd[c], off, 64);
        }
        if (lane == 0)
            for (int c = 0; c < 3; ++c) a.directed_forces[3 * e + c] -= fd[c];
    }
}

bool valid_radial(const SymmetrixJitHipRadialSplineV1& s)
{
    return s.struct_size >= sizeof(SymmetrixJitHipRadialSplineV1) && s.edge_types > 0 && s.intervals > 0 &&
           s.functions >= static_cast<uint32_t>(NP * C) && std::isfinite(s.h) && s.h > 0.0 && std::isfinite(s.x0) &&
           s.coefficients != nullptr;
}

int32_t grid(int64_t items, int32_t persistent_blocks)
{
    return static_cast<int32_t>(items < persistent_blocks ? items : persistent_blocks);
}

int32_t r1_forward_launch(const SymmetrixJitHipR1ForwardArgsV1* args, void* stream, int32_t persistent_blocks)
{
    if (args == nullptr || args->struct_size < sizeof(SymmetrixJitHipR1ForwardArgsV1) ||
        !valid_radial(args->radial) || args->num_nodes < 0 || args->num_nodes > INT32_MAX || args->num_edges < 0 ||
        args->num_edges > INT32_MAX || !std::isfinite(args->cutoff) || args->cutoff <= 0.0 ||
        args->active_type_count == 0 || persistent_blocks <= 0)
        return static_cast<int32_t>(hipErrorInvalidValue);
    if (args->num_nodes == 0) return static_cast<int32_t>(hipSuccess);
    forward_kernel<<<grid(args->num_nodes, persistent_blocks), kForwardThreads, 0,
                     static_cast<hipStream_t>(stream)>>>(*args);
    return static_cast<int32_t>(hipPeekAtLastError());
}

int32_t r1_coordinate_reverse_launch(const SymmetrixJitHipR1SourceArgsV1* source_args,
                                     const SymmetrixJitHipR1EdgeArgsV1* edge_args, void* stream,
                                     int32_t persistent_blocks)
{
    if (source_args == nullptr || edge_args == nullptr ||
        source_args->struct_size < sizeof(SymmetrixJitHipR1SourceArgsV1) ||
        edge_args->struct_size < sizeof(SymmetrixJitHipR1EdgeArgsV1) || !valid_radial(source_args->radial) ||
        !valid_radial(edge_args->radial) || source_args->num_nodes < 0 || source_args->num_nodes > INT32_MAX ||
        source_args->num_edges < 0 || source_args->num_edges > INT32_MAX ||
        source_args->num_edges != edge_args->num_edges ||
        source_args->active_type_count != edge_args->active_type_count || source_args->cutoff != edge_args->cutoff ||
        !std::isfinite(source_args->cutoff) || source_args->cutoff <= 0.0 || source_args->active_type_count == 0 ||
        persistent_blocks <= 0 ||
        (edge_args->coordinates_are_unit && edge_args->coordinate_scalar_size != sizeof(float) &&
         edge_args->coordinate_scalar_size != sizeof(double)))
        return static_cast<int32_t>(hipErrorInvalidValue);
    if (source_args->num_nodes == 0 || source_args->num_edges == 0) return static_cast<int32_t>(hipSuccess);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    source_kernel<<<grid(source_args->num_nodes, persistent_blocks), kSourceThreads, 0, s>>>(*source_args);
    const hipError_t err = hipPeekAtLastError();
    if (err != hipSuccess) return static_cast<int32_t>(err);
    edge_kernel<<<grid((edge_args->num_edges + 3) / 4, persistent_blocks), kEdgeThreads, 0, s>>>(*edge_args);
    return static_cast<int32_t>(hipPeekAtLastError());
}

const SymmetrixJitHipPluginV1 kPlugin = {
    SYMMETRIX_JIT_HIP_PLUGIN_ABI_VERSION_V1,
    sizeof(SymmetrixJitHipPluginV1),
    sizeof(void*),
    SYMMETRIX_JIT_HIP_PLUGIN_BYTE_ORDER,
    SYMMETRIX_JIT_HIP_R1_FORWARD_LAUNCH_V1 | SYMMETRIX_JIT_HIP_R1_COORDINATE_REVERSE_LAUNCH_V1,
    SYMMETRIX_JIT_HIP_SCALAR_FLOAT32_V1,
    sizeof(float),
    0u,
    SYMMETRIX_JIT_HIP_PLUGIN_ABI_TAG_V1,
    "symmetrix-xl-amd/r1/" SXL_R1_PLUGIN_NAME "/gfx950",
    sxl_r1_plugin::kContractFingerprint,
    sxl_r1_plugin::kSemanticFingerprint,
    sxl_r1_plugin::kStructureFingerprint,
    C,
    sxl_r1_plugin::kEmbedding,
    SXL_R1_PLUGIN_EDGE_LMAX,
    SXL_R1_PLUGIN_SOURCE_LMAX,
    "gfx950",
    "",
    64,
    kForwardThreads,
    kSourceThreads,
    kEdgeThreads,
    kPersistentBlocksPerCU,
    &r1_forward_launch,
    &r1_coordinate_reverse_launch,
};

}  // namespace

extern "C" __attribute__((visibility("default"))) const SymmetrixJitHipPluginV1* symmetrix_jit_hip_plugin_query_v1(void)
{
    return &kPlugin;
}
