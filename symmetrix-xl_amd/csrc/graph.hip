// Device graph construction: periodic cell-binned neighbour search, scans,
// the receiver array and the deterministic source-major transpose.
//
// The neighbour search follows the reference's device algorithm
// (libsymmetrix/source/neighbor_graph_kokkos.cpp:117-402): wrap to fractional
// [0,1), bin, sort each bin ascending, and for every receiver walk the
// dz -> dy -> dx stencil and each bin's atoms in ascending order, skipping the
// self image and keeping d^2 <= cutoff^2.  Floating-point contraction is off
// in this file (and the build passes -ffp-contract=off), so the double
// arithmetic rounds exactly like the CPU restatement and the edge list is
// bit-identical to it.
#pragma clang fp contract(off)

#include <hip/hip_runtime.h>

#include <algorithm>
#include <limits>
#include <mutex>
#include <stdexcept>
#include <string>

#include "../../include/symmetrix_amd.h"
#include "evaluator.hpp"
#include "kernels.hpp"

namespace sxl {
namespace {

__device__ __forceinline__ int floor_div(int numerator, int denominator)
{
    const int quotient = numerator / denominator;
    const int remainder = numerator % denominator;
    return quotient - ((remainder != 0 && remainder < 0) ? 1 : 0);
}

__global__ void bins_kernel(NeighborPlan p, const double* __restrict__ pos, double* __restrict__ rf,
                            double* __restrict__ wp, double* __restrict__ wf, int* __restrict__ wrap,
                            int* __restrict__ atom_bins, int* __restrict__ bin_sizes)
{
    const int atom = blockIdx.x * blockDim.x + threadIdx.x;
    if (atom >= p.num_nodes) return;
    double fractional[3];
    for (int axis = 0; axis < 3; ++axis) {
        double value = 0.0;
        for (int component = 0; component < 3; ++component)
            value += pos[3 * static_cast<size_t>(atom) + component] * p.inverse_cell[3 * component + axis];
        rf[3 * static_cast<size_t>(atom) + axis] = value;
        const int w = static_cast<int>(floor(value));
        value -= w;
        fractional[axis] = value;
        wf[3 * static_cast<size_t>(atom) + axis] = value;
        wrap[3 * static_cast<size_t>(atom) + axis] = w;
    }
    for (int component = 0; component < 3; ++component) {
        double value = 0.0;
        for (int axis = 0; axis < 3; ++axis) value += fractional[axis] * p.cell[3 * axis + component];
        wp[3 * static_cast<size_t>(atom) + component] = value;
    }
    const int x = min(p.bins[0] - 1, static_cast<int>(fractional[0] * p.bins[0]));
    const int y = min(p.bins[1] - 1, static_cast<int>(fractional[1] * p.bins[1]));
    const int z = min(p.bins[2] - 1, static_cast<int>(fractional[2] * p.bins[2]));
    const int bin = static_cast<int>((static_cast<size_t>(z) * p.bins[1] + y) * p.bins[0] + x);
    atom_bins[atom] = bin;
    atomicAdd(&bin_sizes[bin], 1);
}

__global__ void fill_bins_kernel(int n, const int* __restrict__ atom_bins, int* __restrict__ cursors,
                                 int* __restrict__ bin_atoms)
{
    const int atom = blockIdx.x * blockDim.x + threadIdx.x;
    if (atom >= n) return;
    const int index = atomicAdd(&cursors[atom_bins[atom]], 1);
    bin_atoms[index] = atom;
}

// One wave per receiver: the stencil cells are visited in order
// (dz -> dy -> dx), the atoms of a cell are tested 64 at a time, and the
// accepted ones are placed by ballot and lane prefix count, so every
// receiver's edges come out in the same order as one thread walking the
// cells and their (sorted) atoms one by one.  A launch covers receivers
// [receiver_begin, receiver_begin + receiver_count).  The count pass
// (o.offsets null) stores the number of edges, the largest cell-shift
// component, and with o.last_tile the number of distinct sources the launch
// adds to tile o.tile (launches of consecutive tiles in stream order: a
// source is new to the tile when it last appeared in an earlier one); the
// fill pass writes the edges.
constexpr int kEdgeThreads = 256;

__global__ void __launch_bounds__(kEdgeThreads) edges_kernel(
    NeighborPlan p, const double* __restrict__ wp, const double* __restrict__ wf, const int* __restrict__ wrap,
    const int* __restrict__ atom_bins, const int* __restrict__ bin_offsets, const int* __restrict__ bin_atoms,
    int receiver_begin, int receiver_count, EdgeOutputs o)
{
    const int lane = threadIdx.x & 63;
    const int local_receiver = blockIdx.x * (kEdgeThreads / 64) + (threadIdx.x >> 6);
    if (local_receiver >= receiver_count) return;  // whole wave
    const int receiver = receiver_begin + local_receiver;
    const bool fill = o.offsets != nullptr;
    const int bx = p.bins[0], by = p.bins[1], bz = p.bins[2];
    const int receiver_bin = atom_bins[receiver];
    const int receiver_x = receiver_bin % bx;
    const int receiver_y = (receiver_bin / bx) % by;
    const int receiver_z = static_cast<int>(static_cast<size_t>(receiver_bin) /
                                            (static_cast<size_t>(bx) * static_cast<size_t>(by)));
    long long local = 0;
    const long long out0 = fill ? o.offsets[receiver] : 0;
    int max_shift = 0;
    int new_sources = 0;
    int receiver_wrap[3];
    double rp[3];
    for (int c = 0; c < 3; ++c) {
        rp[c] = wp[3 * static_cast<size_t>(receiver) + c];
        receiver_wrap[c] = wrap[3 * static_cast<size_t>(receiver) + c];
    }
    for (int dz = -p.reach[2]; dz <= p.reach[2]; ++dz) {
        const int raw_z = receiver_z + dz;
        const int shift_z = floor_div(raw_z, bz);
        const int source_z = raw_z - shift_z * bz;
        for (int dy = -p.reach[1]; dy <= p.reach[1]; ++dy) {
            const int raw_y = receiver_y + dy;
            const int shift_y = floor_div(raw_y, by);
            const int source_y = raw_y - shift_y * by;
            for (int dx = -p.reach[0]; dx <= p.reach[0]; ++dx) {
                const int raw_x = receiver_x + dx;
                const int shift_x = floor_div(raw_x, bx);
                const int source_x = raw_x - shift_x * bx;
                const int source_bin = static_cast<int>(
                    (static_cast<size_t>(source_z) * by + source_y) * bx + source_x);
                const int image[3] = {shift_x, shift_y, shift_z};
                const int b0 = bin_offsets[source_bin], b1 = bin_offsets[source_bin + 1];
                for (int base = b0; base < b1; base += 64) {
                    const int index = base + lane;
                    bool accept = false;
                    int source = 0;
                    if (index < b1) {
                        source = bin_atoms[index];
                        if (!(source == receiver && shift_x == 0 && shift_y == 0 && shift_z == 0)) {
                            double distance_squared = 0.0;
                            for (int component = 0; component < 3; ++component) {
                                double displacement = wp[3 * static_cast<size_t>(source) + component] - rp[component];
                                for (int axis = 0; axis < 3; ++axis)
                                    displacement += image[axis] * p.cell[3 * axis + component];
                                distance_squared += displacement * displacement;
                            }
                            accept = !(distance_squared > p.cutoff_squared);
                        }
                    }
                    const unsigned long long mask = __ballot(accept);
                    if (accept) {
                        int shift[3];
                        for (int axis = 0; axis < 3; ++axis)
                            shift[axis] = image[axis] - wrap[3 * static_cast<size_t>(source) + axis] +
                                          receiver_wrap[axis];
                        if (fill) {
                            const int rank = __builtin_amdgcn_mbcnt_hi(
                                static_cast<unsigned>(mask >> 32),
                                __builtin_amdgcn_mbcnt_lo(static_cast<unsigned>(mask), 0));
                            const size_t edge = static_cast<size_t>(out0 + local + rank);
                            o.sources[edge] = source;
                            for (int axis = 0; axis < 3; ++axis) {
                                if (o.shifts8)
                                    o.shifts8[3 * edge + axis] = static_cast<signed char>(shift[axis]);
                                else
                                    o.shifts[3 * edge + axis] = shift[axis];
                                if (o.frac)
                                    o.frac[3 * edge + axis] = wf[3 * static_cast<size_t>(source) + axis] -
                                                              wf[3 * static_cast<size_t>(receiver) + axis] + image[axis];
                            }
                        } else {
                            for (int axis = 0; axis < 3; ++axis)
                                max_shift = max(max_shift, abs(shift[axis]));
                            if (o.last_tile && atomicExch(o.last_tile + source, o.tile) != o.tile) ++new_sources;
                        }
                    }
                    local += __popcll(mask);
                }
            }
        }
    }
    if (!fill) {
        for (int off = 32; off > 0; off >>= 1) {
            max_shift = max(max_shift, __shfl_xor(max_shift, off, 64));
            new_sources += __shfl_xor(new_sources, off, 64);
        }
        if (lane == 0) {
            o.counts[receiver] = local;
            if (o.max_shift && max_shift > 0) atomicMax(o.max_shift, max_shift);
            if (o.last_tile && new_sources > 0) atomicAdd(o.tile_runs, new_sources);
        }
    }
}

// ---- scans ---------------------------------------------------------------
constexpr int kScanThreads = 256;
constexpr int kScanItems = 4;
constexpr int kScanSpan = kScanThreads * kScanItems;

template <typename In>
__global__ void __launch_bounds__(kScanThreads) scan_blocks_kernel(const In* __restrict__ in, int n,
                                                                   long long* __restrict__ out,
                                                                   long long* __restrict__ block_sums)
{
    __shared__ long long s[kScanThreads];
    const int t = threadIdx.x;
    const size_t base = static_cast<size_t>(blockIdx.x) * kScanSpan + static_cast<size_t>(t) * kScanItems;
    long long v[kScanItems];
    long long local = 0;
    for (int q = 0; q < kScanItems; ++q) {
        const size_t idx = base + q;
        v[q] = idx < static_cast<size_t>(n) ? static_cast<long long>(in[idx]) : 0;
        local += v[q];
    }
    s[t] = local;
    __syncthreads();
    for (int off = 1; off < kScanThreads; off <<= 1) {
        const long long add = t >= off ? s[t - off] : 0;
        __syncthreads();
        s[t] += add;
        __syncthreads();
    }
    long long run = s[t] - local;  // exclusive prefix of this thread
    for (int q = 0; q < kScanItems; ++q) {
        const size_t idx = base + q;
        if (idx < static_cast<size_t>(n)) out[idx] = run;
        run += v[q];
    }
    if (t == kScanThreads - 1) block_sums[blockIdx.x] = s[t];
}

// exclusive scan of block sums in place (one workgroup, sequential chunks);
// writes the grand total to *total
__global__ void __launch_bounds__(kScanThreads) scan_sums_kernel(long long* __restrict__ sums, int nb,
                                                                 long long* __restrict__ total)
{
    __shared__ long long s[kScanThreads];
    __shared__ long long carry;
    const int t = threadIdx.x;
    if (t == 0) carry = 0;
    __syncthreads();
    for (int base = 0; base < nb; base += kScanThreads) {
        const int idx = base + t;
        const long long v = idx < nb ? sums[idx] : 0;
        s[t] = v;
        __syncthreads();
        for (int off = 1; off < kScanThreads; off <<= 1) {
            const long long add = t >= off ? s[t - off] : 0;
            __syncthreads();
            s[t] += add;
            __syncthreads();
        }
        if (idx < nb) sums[idx] = carry + s[t] - v;
        __syncthreads();
        if (t == kScanThreads - 1) carry += s[t];
        __syncthreads();
    }
    if (t == 0) *total = carry;
}

__global__ void scan_add_kernel(long long* __restrict__ out, int n, const long long* __restrict__ sums)
{
    const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= static_cast<size_t>(n)) return;
    out[idx] += sums[idx / kScanSpan];
}

template <typename In>
hipError_t exclusive_scan(const In* in, int n, long long* out, long long* scratch, hipStream_t s)
{
    // out has n+1 entries; out[n] = total
    const int nb = n > 0 ? (n + kScanSpan - 1) / kScanSpan : 0;
    if (nb > 0) {
        scan_blocks_kernel<In><<<nb, kScanThreads, 0, s>>>(in, n, out, scratch), note_launch();
        scan_sums_kernel<<<1, kScanThreads, 0, s>>>(scratch, nb, out + n), note_launch();
        scan_add_kernel<<<(n + 255) / 256, 256, 0, s>>>(out, n, scratch), note_launch();
    } else {
        hipError_t err = hipMemsetAsync(out, 0, sizeof(long long), s);
        if (err != hipSuccess) return err;
    }
    return hipGetLastError();
}

__global__ void narrow_kernel(const long long* __restrict__ offsets, int n, int* __restrict__ out,
                              int* __restrict__ counts)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i > n) return;
    out[i] = static_cast<int>(offsets[i]);
    if (counts && i < n) counts[i] = static_cast<int>(offsets[i + 1] - offsets[i]);
}

__global__ void receivers_kernel(int n, const int* __restrict__ first, int* __restrict__ receiver)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    for (int e = first[i]; e < first[i + 1]; ++e) receiver[e] = i;
}

__global__ void transpose_count_kernel(int E, const int* __restrict__ source, int* __restrict__ counts)
{
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    atomicAdd(&counts[source[e]], 1);
}

__global__ void transpose_fill_kernel(int E, const int* __restrict__ source, const int* __restrict__ tfirst,
                                      int* __restrict__ cursors, int* __restrict__ tedge)
{
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const int s = source[e];
    const int slot = atomicAdd(&cursors[s], 1);
    tedge[tfirst[s] + slot] = e;
}

// Ascending sort of each segment: makes atomic fill orders canonical.  One
// wave per segment: the segment is staged in LDS and every element is
// written at its rank (the number of smaller elements, ties by position), so
// the result is the stable ascending order.  A segment longer than the LDS
// stage is sorted in place by lane 0 (insertion sort).
constexpr int kSortThreads = 256;
constexpr int kSortStage = 1024;  // elements staged per wave

__global__ void __launch_bounds__(kSortThreads) sort_segments_kernel(int nseg, const int* __restrict__ offsets,
                                                                     int* __restrict__ values)
{
    __shared__ int stage[kSortThreads / 64][kSortStage];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int sgm = blockIdx.x * (kSortThreads / 64) + wave;
    if (sgm >= nseg) return;  // whole wave: no block barrier follows
    const int begin = offsets[sgm], end = offsets[sgm + 1];
    const int n = end - begin;
    if (n <= 1) return;
    if (n > kSortStage) {
        if (lane == 0) {
            for (int index = begin + 1; index < end; ++index) {
                const int v = values[index];
                int ins = index;
                while (ins > begin && values[ins - 1] > v) {
                    values[ins] = values[ins - 1];
                    --ins;
                }
                values[ins] = v;
            }
        }
        return;
    }
    int* st = stage[wave];
    for (int i = lane; i < n; i += 64) st[i] = values[begin + i];
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    for (int i = lane; i < n; i += 64) {
        const int v = st[i];
        int rank = 0;
        for (int j = 0; j < n; ++j) {
            const int u = st[j];
            rank += (u < v || (u == v && j < i)) ? 1 : 0;
        }
        values[begin + rank] = v;
    }
}

// Displacement of every atom from its reference position (reference
// prepared_atom_displacements, mace_kokkos_factorized_lifecycle.cpp:2986-3023):
// delta = pos - ref (ref = frac_ref cell for fractional reference positions);
// with any periodic axis, f = delta cell^-1, f -= floor(f + 1/2) on the
// periodic axes, disp = f cell; without, disp = delta.  out[0] collects
// max |disp|^2 (as ordered bits; non-finite: infinite).
__global__ void clear_pair_kernel(unsigned long long* __restrict__ out)
{
    if (threadIdx.x < 2) out[threadIdx.x] = 0ull;
}

__global__ void atom_displacements_kernel(int n, const double* __restrict__ pos, GeometryRef g,
                                          const double* __restrict__ cell,
                                          const double* __restrict__ inverse_cell, double* __restrict__ disp,
                                          unsigned long long* __restrict__ out)
{
    __shared__ double s[256];
    const int t = threadIdx.x;
    const double* __restrict__ ref = g.positions;
    double m = 0.0;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + t; i < static_cast<size_t>(n);
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        double delta[3], f[3], d[3];
        for (int c = 0; c < 3; ++c) {
            double reference = ref[3 * i + c];
            if (g.fractional) {
                reference = 0.0;
                for (int axis = 0; axis < 3; ++axis) reference += ref[3 * i + axis] * cell[3 * axis + c];
            }
            delta[c] = pos[3 * i + c] - reference;
        }
        if (g.pbc == 0) {
            for (int c = 0; c < 3; ++c) d[c] = delta[c];
        } else {
            for (int axis = 0; axis < 3; ++axis) {
                double v = 0.0;
                for (int c = 0; c < 3; ++c) v += delta[c] * inverse_cell[3 * c + axis];
                f[axis] = (g.pbc >> axis) & 1 ? v - floor(v + 0.5) : v;
            }
            for (int c = 0; c < 3; ++c) {
                double v = 0.0;
                for (int axis = 0; axis < 3; ++axis) v += f[axis] * cell[3 * axis + c];
                d[c] = v;
            }
        }
        for (int c = 0; c < 3; ++c) disp[3 * i + c] = d[c];
        const double d2 = d[0] * d[0] + d[1] * d[1] + d[2] * d[2];
        m = d2 > m ? d2 : m;
        if (!(d2 == d2) || d2 > 1.0e300) m = __longlong_as_double(0x7ff0000000000000LL);
    }
    s[t] = m;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (t < w) s[t] = s[t + w] > s[t] ? s[t + w] : s[t];
        __syncthreads();
    }
    if (t == 0) atomicMax(out, static_cast<unsigned long long>(__double_as_longlong(s[0])));
}

__global__ void edge_pairs_kernel(int E, const int* __restrict__ receiver, const int* __restrict__ source,
                                  const int* __restrict__ node_types, const int* __restrict__ type_active,
                                  int n, bool shared, int* __restrict__ edge_pair)
{
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const int a = type_active[node_types[receiver[e]]];
    const int b = type_active[node_types[source[e]]];
    const int ordered = a * n + b;
    const int unordered = shared ? 0 : a <= b ? a * (2 * n - a - 1) / 2 + b : b * (2 * n - b - 1) / 2 + a;
    edge_pair[e] = ordered | (unordered << 16);
}

// Source-grouped edge list of one receiver tile.  The tile's launches run
// after those of every earlier tile, so a source whose last_tile entry is
// not this tile has not been seen in it yet: exactly one of its edges wins
// the exchange and opens its run.
__global__ void tile_runs_mark_kernel(int n, const int* __restrict__ sources, int tile, int* __restrict__ last_tile,
                                      int* __restrict__ run_of, int* __restrict__ run_source,
                                      int* __restrict__ run_count)
{
    const int l = blockIdx.x * blockDim.x + threadIdx.x;
    if (l >= n) return;
    const int src = sources[l];
    if (atomicExch(last_tile + src, tile) != tile) {
        const int k = atomicAdd(run_count, 1);
        if (run_source) {  // null: count only
            run_source[k] = src;
            run_of[src] = k;
        }
    }
}

__global__ void tile_runs_length_kernel(int n, const int* __restrict__ sources, const int* __restrict__ run_of,
                                        int* __restrict__ run_length)
{
    const int l = blockIdx.x * blockDim.x + threadIdx.x;
    if (l >= n) return;
    atomicAdd(run_length + run_of[sources[l]], 1);
}

__global__ void tile_list_fill_kernel(int n, const int* __restrict__ sources, const int* __restrict__ run_of,
                                      const int* __restrict__ run_start, int* __restrict__ cursors,
                                      int* __restrict__ list)
{
    const int l = blockIdx.x * blockDim.x + threadIdx.x;
    if (l >= n) return;
    const int k = run_of[sources[l]];
    list[run_start[k] + atomicAdd(cursors + k, 1)] = l;
}

__global__ void fill_i32_range_kernel(int* __restrict__ out, long long n, int value)
{
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) out[i] = value;
}

// ---- caller graphs on the device --------------------------------------------
// flags[0] neighbour index out of range, [1] type out of range, [2] type not
// active, [3] neighbour type differing from its source's type
__global__ void check_neighbors_kernel(int E, int N, const int* __restrict__ source, const int* __restrict__ ntypes,
                                       const int* __restrict__ node_types, const int* __restrict__ type_active,
                                       int num_elements, unsigned long long* __restrict__ flags)
{
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const int s = source[e], t = ntypes[e];
    if (s < 0 || s >= N) {
        atomicAdd(flags, 1ull);
        return;
    }
    if (t < 0 || t >= num_elements) {
        atomicAdd(flags + 1, 1ull);
        return;
    }
    if (type_active[t] < 0) atomicAdd(flags + 2, 1ull);
    if (t != node_types[s]) atomicAdd(flags + 3, 1ull);
}

// ---- LAMMPS KOKKOS neighbour lists (pair style on device arrays) -------------
// flags: [0] ilist entry out of range or repeated, [1] neighbour index out of
// range, [2] LAMMPS type out of range, [3] a neighbour's local atom is not in
// ilist
__global__ void pair_index_kernel(int inum, const int* __restrict__ ilist, int nall, int* __restrict__ ii_from_i,
                                  unsigned* __restrict__ flags)
{
    const int ii = blockIdx.x * blockDim.x + threadIdx.x;
    if (ii >= inum) return;
    const int i = ilist[ii];
    if (i < 0 || i >= nall || atomicExch(ii_from_i + i, ii) != -1) atomicOr(flags, 1u);
}

__device__ __forceinline__ int pair_neighbor(const PairList& p, int i, int jj)
{
    return p.neighbors[static_cast<long long>(i) * p.stride_atom + static_cast<long long>(jj) * p.stride_slot] &
           kNeighMaskDevice;
}

// One wave per list entry ii: the neighbours within r_cut (stable: all
// listed neighbours) are counted, or (offsets set) written in list order --
// neighbour node, its element, the edge vector x_j - x_i and its length -- by
// ballot and lane prefix count.  The length is formed as on the host (no
// fused operations in this file).  A stable fill scales an edge at
// r >= r_cut to length r_cut (reference pair_symmetrix_mace_kokkos.cpp:
// 1134-1150) and, for a geometry update (neigh_indices null), writes only
// within the entry's edges from offsets and flags a count that differs.
__global__ void __launch_bounds__(256) pair_edges_kernel(PairList p, const int* __restrict__ ii_from_i,
                                                         const long long* __restrict__ offsets,
                                                         int* __restrict__ node_types, int* __restrict__ counts,
                                                         int* __restrict__ neigh_indices, int* __restrict__ neigh_types,
                                                         double* __restrict__ xyz, double* __restrict__ r,
                                                         unsigned* __restrict__ flags)
{
    const int lane = threadIdx.x & 63;
    const int ii = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (ii >= p.inum) return;  // whole wave
    const int i = p.ilist[ii];
    if (i < 0 || i >= p.nall) return;  // flagged by pair_index_kernel
    const bool fill = offsets != nullptr;
    const bool geometry_only = fill && neigh_indices == nullptr;
    const double xi = p.x[3 * static_cast<size_t>(i)], yi = p.x[3 * static_cast<size_t>(i) + 1],
                 zi = p.x[3 * static_cast<size_t>(i) + 2];
    const int n = p.numneigh[i];
    long long out = fill ? offsets[ii] : 0;
    const long long room = geometry_only ? offsets[ii + 1] - out : 0;  // the entry's edges at the last rebuild
    int local = 0;
    unsigned bad = 0;
    for (int base = 0; base < n; base += 64) {
        const int jj = base + lane;
        bool accept = false;
        int j = 0;
        double dx = 0.0, dy = 0.0, dz = 0.0, r2 = 0.0;
        if (jj < n) {
            j = pair_neighbor(p, i, jj);
            if (j < 0 || j >= p.nall) {
                bad |= 2u;
            } else {
                dx = p.x[3 * static_cast<size_t>(j)] - xi;
                dy = p.x[3 * static_cast<size_t>(j) + 1] - yi;
                dz = p.x[3 * static_cast<size_t>(j) + 2] - zi;
                r2 = dx * dx + dy * dy + dz * dz;
                accept = p.stable || r2 < p.r_cut_squared;
            }
        }
        if (accept && !fill) {
            const int jl = p.local_of[j];
            if (jl < 0 || jl >= p.nall || ii_from_i[jl] < 0) bad |= 8u;
            const int t = p.type[j];
            if (t < 1 || t > p.ntypes) bad |= 4u;
        }
        const unsigned long long mask = __ballot(accept);
        if (fill && accept) {
            const int rank = __builtin_amdgcn_mbcnt_hi(static_cast<unsigned>(mask >> 32),
                                                       __builtin_amdgcn_mbcnt_lo(static_cast<unsigned>(mask), 0));
            if (!geometry_only || local + rank < room) {
                const size_t e = static_cast<size_t>(out + local + rank);
                if (!geometry_only) {
                    neigh_indices[e] = ii_from_i[p.local_of[j]];
                    neigh_types[e] = p.mace_types[p.type[j] - 1];
                }
                double len = sqrt(r2);
                if (p.stable && !(r2 < p.r_cut_squared)) {
                    const double scale = p.r_cut / len;
                    dx *= scale;
                    dy *= scale;
                    dz *= scale;
                    len = p.r_cut;
                }
                xyz[3 * e] = dx;
                xyz[3 * e + 1] = dy;
                xyz[3 * e + 2] = dz;
                r[e] = len;
            }
        }
        local += __popcll(mask);
    }
    if (geometry_only) {
        for (int off = 32; off > 0; off >>= 1) bad |= __shfl_xor(bad, off, 64);
        if (local != room) bad |= 16u;
        if (lane == 0 && bad) atomicOr(flags, bad);
    }
    if (!fill) {
        for (int off = 32; off > 0; off >>= 1) bad |= __shfl_xor(bad, off, 64);
        if (lane == 0) {
            counts[ii] = local;
            const int t = p.type[i];
            if (t < 1 || t > p.ntypes) bad |= 4u;
            else node_types[ii] = p.mace_types[t - 1];
            if (bad) atomicOr(flags, bad);
        }
    }
}

// f[ilist[ii]] += F[ii] (the node's reduced force) and eatom[ilist[ii]] = E[ii]
__global__ void pair_scatter_kernel(int inum, const int* __restrict__ ilist, const double* __restrict__ node_forces,
                                    const double* __restrict__ node_energies, double* __restrict__ f,
                                    double* __restrict__ eatom)
{
    const int ii = blockIdx.x * blockDim.x + threadIdx.x;
    if (ii >= inum) return;
    const size_t i = ilist[ii];
    for (int c = 0; c < 3; ++c) f[3 * i + c] += node_forces[3 * static_cast<size_t>(ii) + c];
    if (eatom) eatom[i] = node_energies[ii];
}

}  // namespace

hipError_t launch_check_neighbors(long long num_edges, int num_nodes, const int* source, const int* neigh_types,
                                  const int* node_types, const int* type_active, int num_elements,
                                  unsigned long long* flags, hipStream_t s)
{
    if (num_edges <= 0) return hipSuccess;
    check_neighbors_kernel<<<static_cast<unsigned>((num_edges + 255) / 256), 256, 0, s>>>(
        static_cast<int>(num_edges), num_nodes, source, neigh_types, node_types, type_active, num_elements, flags),
        note_launch();
    return hipGetLastError();
}

hipError_t launch_pair_index(int inum, const int* ilist, int nall, int* ii_from_i, unsigned* flags, hipStream_t s)
{
    if (inum <= 0) return hipSuccess;
    pair_index_kernel<<<(inum + 255) / 256, 256, 0, s>>>(inum, ilist, nall, ii_from_i, flags), note_launch();
    return hipGetLastError();
}

hipError_t launch_pair_edges(const PairList& p, const int* ii_from_i, const long long* offsets, int* node_types,
                             int* counts, int* neigh_indices, int* neigh_types, double* xyz, double* r, unsigned* flags,
                             hipStream_t s)
{
    if (p.inum <= 0) return hipSuccess;
    pair_edges_kernel<<<(p.inum + 3) / 4, 256, 0, s>>>(p, ii_from_i, offsets, node_types, counts, neigh_indices,
                                                       neigh_types, xyz, r, flags), note_launch();
    return hipGetLastError();
}

hipError_t launch_pair_scatter(int inum, const int* ilist, const double* node_forces, const double* node_energies,
                               double* f, double* eatom, hipStream_t s)
{
    if (inum <= 0) return hipSuccess;
    pair_scatter_kernel<<<(inum + 255) / 256, 256, 0, s>>>(inum, ilist, node_forces, node_energies, f, eatom),
        note_launch();
    return hipGetLastError();
}

hipError_t launch_edge_pairs(int num_edges, const int* receiver, const int* source, const int* node_types,
                             const int* type_active, int num_active, bool shared_tables, int* edge_pair,
                             hipStream_t s)
{
    if (num_edges <= 0) return hipSuccess;
    edge_pairs_kernel<<<(num_edges + 255) / 256, 256, 0, s>>>(num_edges, receiver, source, node_types,
                                                              type_active, num_active, shared_tables, edge_pair), note_launch();
    return hipGetLastError();
}

hipError_t launch_neighbor_bins(const NeighborPlan& p, const double* positions, double* reference_fractional,
                                double* wrapped_positions, double* wrapped_fractional, int* wrap_shifts,
                                int* atom_bins, int* bin_sizes, hipStream_t s)
{
    if (p.num_nodes <= 0) return hipSuccess;
    bins_kernel<<<(p.num_nodes + 255) / 256, 256, 0, s>>>(p, positions, reference_fractional, wrapped_positions,
                                                          wrapped_fractional, wrap_shifts, atom_bins,
                                                          bin_sizes), note_launch();
    return hipGetLastError();
}

hipError_t launch_neighbor_fill_bins(const NeighborPlan& p, const int* atom_bins, const int* bin_offsets,
                                     int* bin_cursors, int* bin_atoms, hipStream_t s)
{
    (void)bin_offsets;
    if (p.num_nodes <= 0) return hipSuccess;
    fill_bins_kernel<<<(p.num_nodes + 255) / 256, 256, 0, s>>>(p.num_nodes, atom_bins, bin_cursors,
                                                               bin_atoms), note_launch();
    return hipGetLastError();
}

hipError_t launch_neighbor_edges(const NeighborPlan& p, const double* wrapped_positions,
                                 const double* wrapped_fractional, const int* wrap_shifts,
                                 const int* atom_bins, const int* bin_offsets, const int* bin_atoms,
                                 int receiver_begin, int receiver_count, const EdgeOutputs& out, hipStream_t s)
{
    if (receiver_count <= 0) return hipSuccess;
    constexpr int per_block = kEdgeThreads / 64;
    edges_kernel<<<(receiver_count + per_block - 1) / per_block, kEdgeThreads, 0, s>>>(
        p, wrapped_positions, wrapped_fractional, wrap_shifts, atom_bins, bin_offsets, bin_atoms, receiver_begin,
        receiver_count, out), note_launch();
    return hipGetLastError();
}

std::size_t scan_scratch_size(int n) { return static_cast<std::size_t>(n / kScanSpan + 2); }

hipError_t launch_exclusive_scan_i32(const int* in, int n, long long* out, long long* scratch,
                                     hipStream_t s)
{
    return exclusive_scan<int>(in, n, out, scratch, s);
}

hipError_t launch_exclusive_scan_i64(const long long* in, int n, long long* out, long long* scratch,
                                     hipStream_t s)
{
    return exclusive_scan<long long>(in, n, out, scratch, s);
}

hipError_t launch_narrow_offsets(const long long* offsets, int n, int* out_offsets, int* out_counts,
                                 hipStream_t s)
{
    narrow_kernel<<<(n + 1 + 255) / 256, 256, 0, s>>>(offsets, n, out_offsets, out_counts), note_launch();
    return hipGetLastError();
}

hipError_t launch_receivers(int num_nodes, const int* first, int* receiver, hipStream_t s)
{
    if (num_nodes <= 0) return hipSuccess;
    receivers_kernel<<<(num_nodes + 255) / 256, 256, 0, s>>>(num_nodes, first, receiver), note_launch();
    return hipGetLastError();
}

hipError_t launch_transpose_count(int num_edges, const int* source, int* counts, hipStream_t s)
{
    if (num_edges <= 0) return hipSuccess;
    transpose_count_kernel<<<(num_edges + 255) / 256, 256, 0, s>>>(num_edges, source, counts), note_launch();
    return hipGetLastError();
}

hipError_t launch_transpose_fill(int num_edges, const int* source, const int* tfirst, int* cursors,
                                 int* tedge, hipStream_t s)
{
    if (num_edges <= 0) return hipSuccess;
    transpose_fill_kernel<<<(num_edges + 255) / 256, 256, 0, s>>>(num_edges, source, tfirst, cursors,
                                                                  tedge), note_launch();
    return hipGetLastError();
}

hipError_t launch_sort_segments(int num_segments, const int* offsets, int* values, hipStream_t s)
{
    if (num_segments <= 0) return hipSuccess;
    constexpr int per_block = kSortThreads / 64;
    sort_segments_kernel<<<(num_segments + per_block - 1) / per_block, kSortThreads, 0, s>>>(num_segments,
                                                                                           offsets, values), note_launch();
    return hipGetLastError();
}

hipError_t launch_atom_displacements(int n, const double* positions, const GeometryRef& ref, const double* cell,
                                     const double* inverse_cell, double* displacements, double* out, hipStream_t s)
{
    // out[0]: max |disp|^2, out[1]: invalid-edge count of the edge geometry
    // that follows; cleared by a kernel, not a memset, so the sequence can be
    // captured into a replayed HIP graph
    clear_pair_kernel<<<1, 64, 0, s>>>(reinterpret_cast<unsigned long long*>(out)), note_launch();
    hipError_t err = hipGetLastError();
    if (err != hipSuccess || n <= 0) return err;
    const int blocks = std::min((n + 255) / 256, 1024);
    atom_displacements_kernel<<<blocks, 256, 0, s>>>(n, positions, ref, cell, inverse_cell, displacements,
                                                     reinterpret_cast<unsigned long long*>(out)), note_launch();
    return hipGetLastError();
}

hipError_t launch_tile_runs_mark(int tile_edges, const int* sources, int tile, int* last_tile, int* run_of,
                                 int* run_source, int* run_count, hipStream_t s)
{
    if (tile_edges <= 0) return hipSuccess;
    tile_runs_mark_kernel<<<(tile_edges + 255) / 256, 256, 0, s>>>(tile_edges, sources, tile, last_tile, run_of,
                                                                  run_source, run_count), note_launch();
    return hipGetLastError();
}

hipError_t launch_tile_runs_length(int tile_edges, const int* sources, const int* run_of, int* run_length,
                                   hipStream_t s)
{
    if (tile_edges <= 0) return hipSuccess;
    tile_runs_length_kernel<<<(tile_edges + 255) / 256, 256, 0, s>>>(tile_edges, sources, run_of, run_length),
        note_launch();
    return hipGetLastError();
}

hipError_t launch_tile_list_fill(int tile_edges, const int* sources, const int* run_of, const int* run_start,
                                 int* cursors, int* list, hipStream_t s)
{
    if (tile_edges <= 0) return hipSuccess;
    tile_list_fill_kernel<<<(tile_edges + 255) / 256, 256, 0, s>>>(tile_edges, sources, run_of, run_start, cursors,
                                                                  list), note_launch();
    return hipGetLastError();
}

hipError_t launch_fill_i32(int* out, long long n, int value, hipStream_t s)
{
    if (n <= 0) return hipSuccess;
    fill_i32_range_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, s>>>(out, n, value), note_launch();
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Allocation-free neighbour graph (build_periodic_graph_noalloc).  The
// intermediate arrays of the build (wrapped and fractional positions, bins,
// per-receiver counts and offsets, scan partials) are carved from one
// file-scope device array sized for kNoAllocMaxAtoms atoms and
// kNoAllocMaxBins bins.  Host code never uses the array's name as an address:
// each device's copy is found once with hipGetSymbolAddress and that pointer
// is what the kernels receive.  Every region is written before it is read
// (bin sizes are cleared by a fill kernel), so nothing depends on what an
// earlier call left there.
// ---------------------------------------------------------------------------
namespace noalloc {

constexpr std::size_t align256(std::size_t bytes) { return (bytes + 255) / 256 * 256; }
constexpr std::size_t kAtoms = kNoAllocMaxAtoms;
constexpr std::size_t kBins = kNoAllocMaxBins;
constexpr std::size_t kScanParts = (std::max(kAtoms, kBins) + 1) / kScanSpan + 2;
// byte offsets of the regions
constexpr std::size_t kRf = 0;                                           // [N][3] f64
constexpr std::size_t kWp = kRf + align256(kAtoms * 3 * sizeof(double));  // [N][3] f64
constexpr std::size_t kWf = kWp + align256(kAtoms * 3 * sizeof(double));  // [N][3] f64
constexpr std::size_t kWrap = kWf + align256(kAtoms * 3 * sizeof(double));    // [N][3] i32
constexpr std::size_t kAtomBins = kWrap + align256(kAtoms * 3 * sizeof(int));  // [N] i32
constexpr std::size_t kBinAtoms = kAtomBins + align256(kAtoms * sizeof(int));  // [N] i32
constexpr std::size_t kCounts = kBinAtoms + align256(kAtoms * sizeof(int));    // [N] i64
constexpr std::size_t kOffsets = kCounts + align256(kAtoms * sizeof(long long));  // [N+1] i64
constexpr std::size_t kBinSizes = kOffsets + align256((kAtoms + 1) * sizeof(long long));  // [B+1] i32
constexpr std::size_t kBinOff64 = kBinSizes + align256((kBins + 1) * sizeof(int));        // [B+1] i64
constexpr std::size_t kBinOffsets = kBinOff64 + align256((kBins + 1) * sizeof(long long));  // [B+1] i32
constexpr std::size_t kScan = kBinOffsets + align256((kBins + 1) * sizeof(int));            // scan partials
constexpr std::size_t kBytes = kScan + align256(kScanParts * sizeof(long long));

static_assert(kBytes == SXL_NOALLOC_SCRATCH_BYTES && kAtoms == SXL_NOALLOC_MAX_ATOMS && kBins == SXL_NOALLOC_MAX_BINS,
              "the C header states the allocation-free builder's limits and array size");

}  // namespace noalloc

}  // namespace sxl

// the allocation-free builder's working memory, one copy per device
static __device__ __align__(256) unsigned char scratch[sxl::noalloc::kBytes];

namespace sxl {
namespace {

__global__ void fill_i32_kernel(int* __restrict__ out, int n, int value)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = value;
}

__global__ void copy_i32_kernel(int* __restrict__ out, const int* __restrict__ in, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = in[i];
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
unsigned char* g_scratch_address[kMaxDevices] = {};

// Device address of the current device's copy of `scratch`, looked up once
// per device with that device current.
unsigned char* scratch_address()
{
    int device = 0;
    hipError_t err = hipGetDevice(&device);
    if (err != hipSuccess) throw std::runtime_error(std::string("hipGetDevice: ") + hipGetErrorString(err));
    if (device < 0 || device >= kMaxDevices) throw std::runtime_error("device index beyond the scratch table");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_address[device]) {
        void* p = nullptr;
        err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess || !p)
            throw std::runtime_error(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(err));
        g_scratch_address[device] = static_cast<unsigned char*>(p);
    }
    return g_scratch_address[device];
}

void launch_check(hipError_t err, const char* what)
{
    if (err != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(err));
}

}  // namespace

std::size_t noalloc_scratch_bytes() { return noalloc::kBytes; }

void build_periodic_graph_noalloc(const double* d_positions, int num_nodes, const double* cell,
                                  const double* inverse_cell, double cutoff, long long edge_capacity,
                                  int* d_receiver_offsets, int* d_sources, int* d_shifts, double* d_fractional_xyz,
                                  long long* num_edges, hipStream_t s)
{
    const NeighborPlan plan = neighbor_plan(num_nodes, cell, inverse_cell, cutoff);
    const int N = num_nodes;
    const int B = neighbor_plan_bins(plan);
    if (N > kNoAllocMaxAtoms)
        throw std::length_error("allocation-free neighbor graph holds at most " + std::to_string(kNoAllocMaxAtoms) +
                                " atoms (got " + std::to_string(N) + ")");
    if (B > kNoAllocMaxBins)
        throw std::length_error("allocation-free neighbor graph holds at most " + std::to_string(kNoAllocMaxBins) +
                                " cell bins (the cell needs " + std::to_string(B) + ")");
    if (edge_capacity < 0) throw std::invalid_argument("edge capacity must be non-negative");
    if (N == 0) {
        // no atoms, no edges: receiver_offsets = [0]
        fill_i32_kernel<<<1, 64, 0, s>>>(d_receiver_offsets, 1, 0), note_launch();
        launch_check(hipGetLastError(), "neighbor graph");
        launch_check(host_fence(s), "neighbor graph");
        *num_edges = 0;
        return;
    }
    unsigned char* base = scratch_address();
    double* rf = reinterpret_cast<double*>(base + noalloc::kRf);
    double* wp = reinterpret_cast<double*>(base + noalloc::kWp);
    double* wf = reinterpret_cast<double*>(base + noalloc::kWf);
    int* wrap = reinterpret_cast<int*>(base + noalloc::kWrap);
    int* atom_bins = reinterpret_cast<int*>(base + noalloc::kAtomBins);
    int* bin_atoms = reinterpret_cast<int*>(base + noalloc::kBinAtoms);
    long long* counts = reinterpret_cast<long long*>(base + noalloc::kCounts);
    long long* offsets = reinterpret_cast<long long*>(base + noalloc::kOffsets);
    int* bin_sizes = reinterpret_cast<int*>(base + noalloc::kBinSizes);
    long long* bin_off64 = reinterpret_cast<long long*>(base + noalloc::kBinOff64);
    int* bin_offsets = reinterpret_cast<int*>(base + noalloc::kBinOffsets);
    long long* scan = reinterpret_cast<long long*>(base + noalloc::kScan);

    fill_i32_kernel<<<(B + 1 + 255) / 256, 256, 0, s>>>(bin_sizes, B + 1, 0), note_launch();
    launch_check(hipGetLastError(), "clear bins");
    launch_check(launch_neighbor_bins(plan, d_positions, rf, wp, wf, wrap, atom_bins, bin_sizes, s), "bins");
    launch_check(launch_exclusive_scan_i32(bin_sizes, B, bin_off64, scan, s), "bin scan");
    launch_check(launch_narrow_offsets(bin_off64, B, bin_offsets, nullptr, s), "narrow");
    // cursors start at the bin offsets
    copy_i32_kernel<<<(B + 255) / 256, 256, 0, s>>>(bin_sizes, bin_offsets, B), note_launch();
    launch_check(hipGetLastError(), "cursors");
    launch_check(launch_neighbor_fill_bins(plan, atom_bins, bin_offsets, bin_sizes, bin_atoms, s), "fill bins");
    launch_check(launch_sort_segments(B, bin_offsets, bin_atoms, s), "sort bins");
    {
        EdgeOutputs o;
        o.counts = counts;
        launch_check(launch_neighbor_edges(plan, wp, wf, wrap, atom_bins, bin_offsets, bin_atoms, 0, N, o, s),
                     "count edges");
    }
    launch_check(launch_exclusive_scan_i64(counts, N, offsets, scan, s), "edge scan");
    long long total = 0;
    launch_check(hipMemcpyAsync(&total, offsets + N, sizeof(long long), hipMemcpyDeviceToHost, s), "edge count");
    launch_check(host_fence(s), "edge count");
    *num_edges = total;
    if (total > std::numeric_limits<int>::max())
        throw std::length_error("neighbor graph exceeds 32-bit edge indexing");
    if (total > edge_capacity)
        throw std::length_error("neighbor graph has " + std::to_string(total) + " edges, more than the capacity " +
                                std::to_string(edge_capacity) + " of the output arrays");
    launch_check(launch_narrow_offsets(offsets, N, d_receiver_offsets, nullptr, s), "narrow");
    {
        EdgeOutputs o;
        o.offsets = offsets;
        o.sources = d_sources;
        o.shifts = d_shifts;
        o.frac = d_fractional_xyz;
        launch_check(launch_neighbor_edges(plan, wp, wf, wrap, atom_bins, bin_offsets, bin_atoms, 0, N, o, s),
                     "fill edges");
    }
    launch_check(host_fence(s), "neighbor graph");
}

}  // namespace sxl
