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
// direction u = (z, x, y)/r, block l, as homogeneous polynomials of degree l,
// and the gradients of those polynomials with respect to u.
template <int L, bool GRAD>
__device__ __forceinline__ void harmonic_block(float x, float y, float z, float* v, float* gx, float* gy,
                                               float* gz)
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
    if constexpr (L == 0) {
        v[0] = c00;
        if (GRAD) gx[0] = gy[0] = gz[0] = 0.0f;
    } else if constexpr (L == 1) {
        v[0] = c1 * y;
        v[1] = c1 * z;
        v[2] = c1 * x;
        if (GRAD) {
            gx[0] = 0.0f, gy[0] = c1, gz[0] = 0.0f;
            gx[1] = 0.0f, gy[1] = 0.0f, gz[1] = c1;
            gx[2] = c1, gy[2] = 0.0f, gz[2] = 0.0f;
        }
    } else if constexpr (L == 2) {
        const float xx = x * x, yy = y * y, zz = z * z;
        v[0] = c2a * x * y;
        v[1] = c2a * y * z;
        v[2] = c20 * (2.0f * zz - xx - yy);
        v[3] = c2a * x * z;
        v[4] = c22 * (xx - yy);
        if (GRAD) {
            gx[0] = c2a * y, gy[0] = c2a * x, gz[0] = 0.0f;
            gx[1] = 0.0f, gy[1] = c2a * z, gz[1] = c2a * y;
            gx[2] = -2.0f * c20 * x, gy[2] = -2.0f * c20 * y, gz[2] = 4.0f * c20 * z;
            gx[3] = c2a * z, gy[3] = 0.0f, gz[3] = c2a * x;
            gx[4] = 2.0f * c22 * x, gy[4] = -2.0f * c22 * y, gz[4] = 0.0f;
        }
    } else {
        static_assert(L == 3, "harmonic blocks up to l = 3");
        const float xx = x * x, yy = y * y, zz = z * z;
        v[0] = c33 * y * (3.0f * xx - yy);
        v[1] = c32 * x * y * z;
        v[2] = c31 * y * (4.0f * zz - xx - yy);
        v[3] = c30 * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);
        v[4] = c31 * x * (4.0f * zz - xx - yy);
        v[5] = 0.5f * c32 * z * (xx - yy);
        v[6] = c33 * x * (xx - 3.0f * yy);
        if (GRAD) {
            gx[0] = 6.0f * c33 * x * y, gy[0] = 3.0f * c33 * (xx - yy), gz[0] = 0.0f;
            gx[1] = c32 * y * z, gy[1] = c32 * x * z, gz[1] = c32 * x * y;
            gx[2] = -2.0f * c31 * x * y, gy[2] = c31 * (4.0f * zz - xx - 3.0f * yy),
            gz[2] = 8.0f * c31 * y * z;
            gx[3] = -6.0f * c30 * x * z, gy[3] = -6.0f * c30 * y * z,
            gz[3] = c30 * (6.0f * zz - 3.0f * xx - 3.0f * yy);
            gx[4] = c31 * (4.0f * zz - 3.0f * xx - yy), gy[4] = -2.0f * c31 * x * y,
            gz[4] = 8.0f * c31 * x * z;
            gx[5] = c32 * x * z, gy[5] = -c32 * y * z, gz[5] = 0.5f * c32 * (xx - yy);
            gx[6] = 3.0f * c33 * (xx - yy), gy[6] = -6.0f * c33 * x * y, gz[6] = 0.0f;
        }
    }
}

// Block l of the MACE harmonics of the unit direction u (Cartesian) and, with
// GRAD, their gradients d/d(x,y,z) for |r| = 1/ir; written to Y[lm] and
// dY{x,y,z}[lm], lm = l^2 .. (l+1)^2 - 1.
template <int L, bool GRAD>
__device__ __forceinline__ void harmonic_block_out(float ux, float uy, float uz, float ir, float* Y,
                                                   float* dYx, float* dYy, float* dYz)
{
    constexpr int M = 2 * L + 1;
    float v[M], g0[M], g1[M], g2[M];
    // permuted direction (z, x, y)
    harmonic_block<L, GRAD>(uz, ux, uy, v, g0, g1, g2);
#pragma unroll
    for (int m = 0; m < M; ++m) {
        Y[L * L + m] = kShNorm * v[m];
        if constexpr (GRAD) {
            const float lv = static_cast<float>(L) * v[m];
            // d/dx <- d/du1, d/dy <- d/du2, d/dz <- d/du0
            dYx[L * L + m] = kShNorm * (g1[m] - lv * ux) * ir;
            dYy[L * L + m] = kShNorm * (g2[m] - lv * uy) * ir;
            dYz[L * L + m] = kShNorm * (g0[m] - lv * uz) * ir;
        }
    }
}

// MACE harmonics Y[lm] of an edge vector (x,y,z) with length r, and
// optionally dY/d(x,y,z) (unpermuted Cartesian components).  The outputs may
// point into LDS: each l block is stored as soon as it is formed.
template <int LMAX, bool GRAD>
__device__ __forceinline__ void edge_harmonics(const double* xyz, double r, float* Y, float* dYx,
                                               float* dYy, float* dYz, float* dir)
{
    const double inv = 1.0 / r;
    const float ux = static_cast<float>(xyz[0] * inv);
    const float uy = static_cast<float>(xyz[1] * inv);
    const float uz = static_cast<float>(xyz[2] * inv);
    dir[0] = ux;
    dir[1] = uy;
    dir[2] = uz;
    const float ir = static_cast<float>(inv);
    harmonic_block_out<0, GRAD>(ux, uy, uz, ir, Y, dYx, dYy, dYz);
    if constexpr (LMAX >= 1) harmonic_block_out<1, GRAD>(ux, uy, uz, ir, Y, dYx, dYy, dYz);
    if constexpr (LMAX >= 2) harmonic_block_out<2, GRAD>(ux, uy, uz, ir, Y, dYx, dYy, dYz);
    if constexpr (LMAX >= 3) harmonic_block_out<3, GRAD>(ux, uy, uz, ir, Y, dYx, dYy, dYz);
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

// Channel-sliced receivers: `slices` (1, 2, 4 or 8) workgroups per receiver,
// one per channel slice.  Block b runs slice b % slices -- so every XCD
// (b % 8) runs one slice only and its L2 holds that slice's columns of the
// coefficient tables -- of a receiver from a contiguous range per XCD of the
// group of 8 / slices XCDs that run the slice.  Blocks 0 .. slices * count - 1
// cover every (receiver, slice) once.
__device__ __forceinline__ int xcd_slice_receiver(int block, int count, int slices, int& slice)
{
    slice = block % slices;
    const int groups = 8 / slices;
    const int b = block / slices;
    const int x = b % groups;
    const int q = b / groups;
    const int base = count / groups;
    const int rem = count % groups;
    return x * base + min(x, rem) + q;
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_moved(float v)
{
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf, false));
}

// Sum over the 64 lanes of a wave with DPP moves (quad permutes, row
// mirrors, row broadcasts), returned wave-uniform.  Fixed combination order,
// so the result is run-to-run identical.
__device__ __forceinline__ float wave_sum_dpp(float v)
{
    v += dpp_moved<0xb1>(v);         // quad_perm [1,0,3,2]
    v += dpp_moved<0x4e>(v);         // quad_perm [2,3,0,1]
    v += dpp_moved<0x141>(v);        // row_half_mirror
    v += dpp_moved<0x140>(v);        // row_mirror
    v += dpp_moved<0x142, 0xa>(v);   // row_bcast:15 into rows 1 and 3
    v += dpp_moved<0x143, 0xc>(v);   // row_bcast:31 into rows 2 and 3
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Partial wave sums for values the caller stores and adds up itself.  With
// PARTS = 4 the reduction stops within rows of 16 lanes (lanes 15, 31, 47 and
// 63 hold the four row sums); with PARTS = 2 one row broadcast follows (lanes
// 31 and 63 hold the sums of lanes 0..31 and 32..63); with PARTS = 1 lane 63
// holds the wave sum.  The row broadcasts carry a row mask, so each costs a
// zeroed register, a move and an add: stopping early saves them.
template <int PARTS>
__device__ __forceinline__ float partial_sum_dpp(float v)
{
    static_assert(PARTS == 1 || PARTS == 2 || PARTS == 4, "1, 2 or 4 partial sums per wave");
    v += dpp_moved<0xb1>(v);
    v += dpp_moved<0x4e>(v);
    v += dpp_moved<0x141>(v);
    v += dpp_moved<0x140>(v);
    if constexpr (PARTS <= 2) v += dpp_moved<0x142, 0xa>(v);
    if constexpr (PARTS == 1) v += dpp_moved<0x143, 0xc>(v);
    return v;
}

// The lane that holds partial `lane / (64 / PARTS)` of partial_sum_dpp.
template <int PARTS>
__device__ __forceinline__ bool holds_partial(int lane)
{
    return (lane & (64 / PARTS - 1)) == 64 / PARTS - 1;
}

// Wave sums of twelve values, f[c][d] = component c of item d, in 30 VALU
// operations instead of 4-5 DPP steps per value.  v_permlane32_swap
// exchanges the upper half of one register with the lower half of another,
// so adding the pair sums each value over the two lane halves while the
// halves take different values; v_permlane16_swap does the same for the odd
// and even 16-lane rows.  After the two exchanges row r of out[c] holds
// item r's component c summed over lanes congruent mod 16, and a row
// reduction leaves item r's three wave sums in lane 16 r + 15.  The values
// enter in the order v[4c + s(d)], s = (0, 2, 1, 3), which the row exchange
// undoes.  Fixed combination order: run-to-run identical.
//
// Both results of a swap pass through an empty asm statement before they are
// read as floats: this compiler (ROCm 7.2 clang) otherwise folds the float
// view of the second result into the first and adds the first to itself.
__device__ __forceinline__ float swap_pair_sum(unsigned lo, unsigned hi)
{
    asm volatile("" : "+v"(lo), "+v"(hi));
    return __builtin_bit_cast(float, lo) + __builtin_bit_cast(float, hi);
}

__device__ __forceinline__ void wave_sum_3x4(const float (&f)[3][4], float (&out)[3])
{
    constexpr int s[4] = {0, 2, 1, 3};
    float v[12];
#pragma unroll
    for (int c = 0; c < 3; ++c)
#pragma unroll
        for (int d = 0; d < 4; ++d) v[4 * c + s[d]] = f[c][d];
    float w[6];
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        const auto x = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v[2 * i]),
                                                        __builtin_bit_cast(unsigned, v[2 * i + 1]), false, false);
        w[i] = swap_pair_sum(x[0], x[1]);
    }
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const auto x = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, w[2 * c]),
                                                        __builtin_bit_cast(unsigned, w[2 * c + 1]), false, false);
        float u = swap_pair_sum(x[0], x[1]);
        u += dpp_moved<0xb1>(u);   // quad_perm [1,0,3,2]
        u += dpp_moved<0x4e>(u);   // quad_perm [2,3,0,1]
        u += dpp_moved<0x141>(u);  // row_half_mirror
        u += dpp_moved<0x140>(u);  // row_mirror
        out[c] = u;
    }
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ float uniform(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}

// Raw (untyped) buffer resource over [base, base + bytes); gfx9 word 3.
// Loads beyond `bytes` return zero and stores beyond it are dropped.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

typedef float float4v __attribute__((ext_vector_type(4)));

// The raw buffer builtins move untyped 32-bit words (unsigned int); the
// float views are bit casts, never value conversions.
__device__ __forceinline__ float4v load4(__amdgpu_buffer_rsrc_t r, int voffset, int soffset)
{
    return __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(r, voffset, soffset, 0));
}

__device__ __forceinline__ float load1(__amdgpu_buffer_rsrc_t r, int voffset, int soffset)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voffset, soffset, 0));
}

__device__ __forceinline__ void store1(float v, __amdgpu_buffer_rsrc_t r, int voffset, int soffset)
{
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned int, v), r, voffset, soffset, 0);
}

// Non-temporal (streaming) store: cache-policy NT, for data written once and
// read once much later by another kernel, far more than the L2s hold.
constexpr int kCachePolicyNT = 2;
__device__ __forceinline__ void store1_stream(float v, __amdgpu_buffer_rsrc_t r, int voffset, int soffset)
{
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned int, v), r, voffset, soffset, kCachePolicyNT);
}

// Cubic of one interval, c = (c0, c1, c2, c3) in local coordinate x.
__device__ __forceinline__ float cubic(const float4v& c, float x)
{
    return fmaf(x, fmaf(x, fmaf(x, c.w, c.z), c.y), c.x);
}

__device__ __forceinline__ float cubic_slope(const float4v& c, float x, float x3)
{
    return fmaf(x, fmaf(x3, c.w, c.z + c.z), c.y);
}

// Value and slope of the cubic sharing its Horner terms: with
// t1 = c2 + x c3 and t2 = c1 + x t1, value = c0 + x t2 and
// slope = t2 + x (t1 + x c3) = c1 + 2 c2 x + 3 c3 x^2 (five FMAs).
__device__ __forceinline__ void cubic_value_slope(const float4v& c, float x, float& value, float& slope)
{
    const float t1 = fmaf(x, c.w, c.z);
    const float t2 = fmaf(x, t1, c.y);
    value = fmaf(x, t2, c.x);
    slope = fmaf(x, fmaf(x, c.w, t1), t2);
}

__device__ __forceinline__ int unordered_pair(int a, int b, int n)
{
    return a <= b ? a * (2 * n - a - 1) / 2 + b : b * (2 * n - b - 1) / 2 + a;
}

}  // namespace sxl
