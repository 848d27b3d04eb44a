// Device helpers shared by the layer kernels: edge harmonics, spline points,
// receiver-to-workgroup mapping and wave reductions.
#pragma once

#include <hip/hip_runtime.h>

#include "kernels.hpp"

namespace sxl {

// 2*sqrt(pi): MACE normalisation of the orthonormal harmonics
// (reference spherical_harmonic_device.hpp:15-16).
constexpr float kShNorm = 3.5449077018110318f;

// Real harmonics (orthonormal, no Condon-Shortley phase) of the permuted unit
// direction u = (z, x, y)/r, as homogeneous polynomials of degree l, and the
// gradients of those polynomials with respect to u.
template <int LMAX, bool GRAD>
__device__ __forceinline__ void harmonic_forms(float x, float y, float z, float* v, float* gx,
                                               float* gy, float* gz)
{
    constexpr float c00 = 0.28209479177387814f;
    constexpr float c1 = 0.4886025119029199f;
    constexpr float c2a = 1.0925484305920792f;
    constexpr float c20 = 0.31539156525252005f;
    constexpr float c22 = 0.5462742152960396f;
    constexpr float c33 = 0.5900435899266435f;
    constexpr float c32 = 2.890611442640554f;
    constexpr float c31 = 0.4570457994644658f;
    constexpr float c30 = 0.3731763325901154f;
    v[0] = c00;
    if (GRAD) gx[0] = gy[0] = gz[0] = 0.0f;
    if constexpr (LMAX >= 1) {
        v[1] = c1 * y;
        v[2] = c1 * z;
        v[3] = c1 * x;
        if (GRAD) {
            gx[1] = 0.0f, gy[1] = c1, gz[1] = 0.0f;
            gx[2] = 0.0f, gy[2] = 0.0f, gz[2] = c1;
            gx[3] = c1, gy[3] = 0.0f, gz[3] = 0.0f;
        }
    }
    if constexpr (LMAX >= 2) {
        const float xx = x * x, yy = y * y, zz = z * z;
        v[4] = c2a * x * y;
        v[5] = c2a * y * z;
        v[6] = c20 * (2.0f * zz - xx - yy);
        v[7] = c2a * x * z;
        v[8] = c22 * (xx - yy);
        if (GRAD) {
            gx[4] = c2a * y, gy[4] = c2a * x, gz[4] = 0.0f;
            gx[5] = 0.0f, gy[5] = c2a * z, gz[5] = c2a * y;
            gx[6] = -2.0f * c20 * x, gy[6] = -2.0f * c20 * y, gz[6] = 4.0f * c20 * z;
            gx[7] = c2a * z, gy[7] = 0.0f, gz[7] = c2a * x;
            gx[8] = 2.0f * c22 * x, gy[8] = -2.0f * c22 * y, gz[8] = 0.0f;
        }
    }
    if constexpr (LMAX >= 3) {
        const float xx = x * x, yy = y * y, zz = z * z;
        v[9] = c33 * y * (3.0f * xx - yy);
        v[10] = c32 * x * y * z;
        v[11] = c31 * y * (4.0f * zz - xx - yy);
        v[12] = c30 * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);
        v[13] = c31 * x * (4.0f * zz - xx - yy);
        v[14] = 0.5f * c32 * z * (xx - yy);
        v[15] = c33 * x * (xx - 3.0f * yy);
        if (GRAD) {
            gx[9] = 6.0f * c33 * x * y, gy[9] = 3.0f * c33 * (xx - yy), gz[9] = 0.0f;
            gx[10] = c32 * y * z, gy[10] = c32 * x * z, gz[10] = c32 * x * y;
            gx[11] = -2.0f * c31 * x * y, gy[11] = c31 * (4.0f * zz - xx - 3.0f * yy),
            gz[11] = 8.0f * c31 * y * z;
            gx[12] = -6.0f * c30 * x * z, gy[12] = -6.0f * c30 * y * z,
            gz[12] = c30 * (6.0f * zz - 3.0f * xx - 3.0f * yy);
            gx[13] = c31 * (4.0f * zz - 3.0f * xx - yy), gy[13] = -2.0f * c31 * x * y,
            gz[13] = 8.0f * c31 * x * z;
            gx[14] = c32 * x * z, gy[14] = -c32 * y * z, gz[14] = 0.5f * c32 * (xx - yy);
            gx[15] = 3.0f * c33 * (xx - yy), gy[15] = -6.0f * c33 * x * y, gz[15] = 0.0f;
        }
    }
}

// MACE harmonics Y[lm] of an edge vector (x,y,z) with length r, and
// optionally dY/d(x,y,z) (unpermuted Cartesian components).
template <int LMAX, bool GRAD>
__device__ __forceinline__ void edge_harmonics(const double* xyz, double r, float* Y, float* dYx,
                                               float* dYy, float* dYz, float* dir)
{
    constexpr int NLM = (LMAX + 1) * (LMAX + 1);
    const double inv = 1.0 / r;
    const float ux = static_cast<float>(xyz[0] * inv);
    const float uy = static_cast<float>(xyz[1] * inv);
    const float uz = static_cast<float>(xyz[2] * inv);
    dir[0] = ux;
    dir[1] = uy;
    dir[2] = uz;
    float v[NLM], g0[NLM], g1[NLM], g2[NLM];
    // permuted direction (z, x, y)
    harmonic_forms<LMAX, GRAD>(uz, ux, uy, v, g0, g1, g2);
    const float ir = static_cast<float>(inv);
#pragma unroll
    for (int l = 0; l <= LMAX; ++l)
#pragma unroll
        for (int lm = l * l; lm < (l + 1) * (l + 1); ++lm) {
            Y[lm] = kShNorm * v[lm];
            if constexpr (GRAD) {
                const float lv = static_cast<float>(l) * v[lm];
                // d/dx <- d/du1, d/dy <- d/du2, d/dz <- d/du0
                dYx[lm] = kShNorm * (g1[lm] - lv * ux) * ir;
                dYy[lm] = kShNorm * (g2[lm] - lv * uy) * ir;
                dYz[lm] = kShNorm * (g0[lm] - lv * uz) * ir;
            }
        }
}

// Cubic Hermite evaluation point (reference cubic_spline_set.cpp:32-47),
// formed in double from the double distance.
__device__ __forceinline__ void spline_point(double r, const SplineGrid& g, int& interval, float& x)
{
    int i = static_cast<int>(floor((r - g.x0) / g.h));
    double xd = r - g.x0 - g.h * i;
    if (i < 0) {
        i = 0;
        xd = 0.0;
    } else if (i >= g.intervals) {
        i = g.intervals - 1;
        xd = g.h;
    }
    interval = i;
    x = static_cast<float>(xd);
}

// Workgroups are dispatched round-robin over the 8 XCDs; give each XCD a
// contiguous range of receivers so that neighbouring receivers (which share
// most of their sources) hit the same L2.
__device__ __forceinline__ int xcd_contiguous(int block, int count)
{
    constexpr int kXcds = 8;
    const int x = block % kXcds;
    const int q = block / kXcds;
    const int base = count / kXcds;
    const int rem = count % kXcds;
    return x * base + min(x, rem) + q;
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ int unordered_pair(int a, int b, int n)
{
    return a <= b ? a * (2 * n - a - 1) / 2 + b : b * (2 * n - b - 1) / 2 + a;
}

}  // namespace sxl
