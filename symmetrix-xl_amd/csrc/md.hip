// Velocity-Verlet integration kernels of the device NVE driver (the
// counterpart of LAMMPS `fix nve` driving `pair_style symmetrix/mace`,
// pair_symmetrix/pair_symmetrix_mace.cpp:309-441, in the reference's capacity
// runs).  Positions, velocities and forces stay in HBM between steps; every
// update is one pass over [N][3] doubles (HBM-bound, 48-72 bytes per atom).
// Contraction is off in this file so each update rounds like the same
// expression evaluated term by term on the host.
#pragma clang fp contract(off)

#include <hip/hip_runtime.h>

#include <algorithm>

#include "kernels.hpp"

namespace sxl {
namespace {

constexpr int kMdThreads = 256;

// v += dtf f inv_m; x += dt v   (inv_m: unit factor / mass, per atom)
__global__ void kick_drift_kernel(int n, double* __restrict__ x, double* __restrict__ v,
                                  const double* __restrict__ f, const double* __restrict__ inv_m, double dtf,
                                  double dt)
{
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<size_t>(n) * 3) return;
    const double vi = v[i] + dtf * f[i] * inv_m[i / 3];
    v[i] = vi;
    x[i] = x[i] + dt * vi;
}

// v += dtf f inv_m, unless a gate is given and *gate <= gate_limit fails
// (the evaluation whose forces f holds ran on a graph that no longer held)
__global__ void kick_kernel(int n, double* __restrict__ v, const double* __restrict__ f,
                            const double* __restrict__ inv_m, double dtf, const double* __restrict__ gate,
                            double gate_limit)
{
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<size_t>(n) * 3) return;
    if (gate && !(*gate <= gate_limit)) return;
    v[i] = v[i] + dtf * f[i] * inv_m[i / 3];
}

// partials[b] = sum over block b's atoms of m |v|^2 (fixed order per block)
__global__ void __launch_bounds__(kMdThreads) kinetic_partial_kernel(int n, const double* __restrict__ v,
                                                                     const double* __restrict__ m,
                                                                     double* __restrict__ partials)
{
    __shared__ double s[kMdThreads];
    const int t = threadIdx.x;
    double acc = 0.0;
    for (size_t a = static_cast<size_t>(blockIdx.x) * kMdThreads + t; a < static_cast<size_t>(n);
         a += static_cast<size_t>(gridDim.x) * kMdThreads) {
        const double vx = v[3 * a], vy = v[3 * a + 1], vz = v[3 * a + 2];
        acc += m[a] * (vx * vx + vy * vy + vz * vz);
    }
    s[t] = acc;
    __syncthreads();
    for (int w = kMdThreads / 2; w > 0; w >>= 1) {
        if (t < w) s[t] += s[t + w];
        __syncthreads();
    }
    if (t == 0) partials[blockIdx.x] = s[0];
}

__global__ void __launch_bounds__(kMdThreads) kinetic_final_kernel(int num_partials,
                                                                   const double* __restrict__ partials,
                                                                   double* __restrict__ out)
{
    __shared__ double s[kMdThreads];
    const int t = threadIdx.x;
    double acc = 0.0;
    for (int b = t; b < num_partials; b += kMdThreads) acc += partials[b];
    s[t] = acc;
    __syncthreads();
    for (int w = kMdThreads / 2; w > 0; w >>= 1) {
        if (t < w) s[t] += s[t + w];
        __syncthreads();
    }
    if (t == 0) out[0] = s[0];
}

int blocks_for(long long work) { return static_cast<int>((work + kMdThreads - 1) / kMdThreads); }

}  // namespace

int md_kinetic_partials(int num_atoms) { return std::max(1, std::min(1024, blocks_for(num_atoms))); }

hipError_t launch_md_kick_drift(int num_atoms, double* x, double* v, const double* f, const double* inv_m,
                                double dtf, double dt, hipStream_t s)
{
    if (num_atoms <= 0) return hipSuccess;
    kick_drift_kernel<<<blocks_for(3LL * num_atoms), kMdThreads, 0, s>>>(num_atoms, x, v, f, inv_m, dtf, dt), note_launch();
    return hipGetLastError();
}

hipError_t launch_md_kick(int num_atoms, double* v, const double* f, const double* inv_m, double dtf,
                          const double* gate, double gate_limit, hipStream_t s)
{
    if (num_atoms <= 0) return hipSuccess;
    kick_kernel<<<blocks_for(3LL * num_atoms), kMdThreads, 0, s>>>(num_atoms, v, f, inv_m, dtf, gate, gate_limit),
        note_launch();
    return hipGetLastError();
}

hipError_t launch_md_kinetic(int num_atoms, const double* v, const double* m, double* partials, int num_partials,
                             double* out, hipStream_t s)
{
    kinetic_partial_kernel<<<num_partials, kMdThreads, 0, s>>>(num_atoms, v, m, partials), note_launch();
    kinetic_final_kernel<<<1, kMdThreads, 0, s>>>(num_partials, partials, out), note_launch();
    return hipGetLastError();
}

}  // namespace sxl
