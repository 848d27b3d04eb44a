// gfx950 kernels of the MACE energy + force evaluation.
//
// Edge stages are receiver-owned: one workgroup per receiver, one thread per
// channel.  The edges of the receiver are processed in tiles: in a tile
// prologue one thread per edge forms the edge's geometry (spline interval,
// harmonics, their gradients, and for the second interaction the products
// cg_t * Y[lm1_t]) into LDS; the channel threads then stream the tile's edges,
// evaluating the radial splines from the coefficient tables and accumulating
// into registers.  No graph-wide edge state is materialised in the forward
// pass; the reverse pass writes the directed force of each edge and, for the
// second interaction, the edge's H1-adjoint contribution (gathered per source
// afterwards in a fixed order, so results are run-to-run deterministic).
//
// Reference semantics (libsymmetrix/source/mace.cpp): compute_A0_streamed
// :1355-1403, compute_Phi1_streamed :2022-2083, reverse_Phi1_streamed
// :2198-2302, reverse_A0_streamed :1485-1559; reductions
// mace_kokkos_evaluate.cpp:48-291.  The node kernels (M0, readout) are in
// nodes.hip.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "device_math.hpp"
#include "kernels.hpp"
#include "r1_shapes.inc"
#include "sh_grad.inc"

namespace sxl {
namespace {

constexpr int kMaxWaves = 4;  // 256 threads
// partial sums per wave of an edge force component, stored in LDS and added
// in double by the edge's thread (fewer DPP steps than a full reduction)
constexpr int kForceParts = 4;
// the path-group passes add into their partials once per pass: one per wave
// (measured: four per wave made the wide shape's reverse 1 % slower)
constexpr int kForcePartsGrouped = 1;

// l of each harmonic index lm (lm = l^2 .. l^2 + 2l), l <= 3
constexpr int kLmL[16] = {0, 1, 1, 1, 2, 2, 2, 2, 2, 3, 3, 3, 3, 3, 3, 3};

__device__ __forceinline__ int receiver_of_block(const LayerArgs& a)
{
    return a.node_offset + xcd_contiguous(blockIdx.x, a.node_count);
}

// Layer-0 receivers in element-type order when the type order is given: the
// workgroups running at any moment (on every XCD) then share the folded
// spline tables of one receiver type, whose rows are per ordered pair.
__device__ __forceinline__ int layer0_receiver(const LayerArgs& a)
{
    return a.type_order ? a.type_order[a.node_offset + blockIdx.x] : receiver_of_block(a);
}

// ---------------------------------------------------------------------------
// Edge tiles.  Wave 0 of the workgroup stages up to 64 edges of the receiver:
// the edges within r_cut are compacted (ballot + lane prefix count) into LDS
// slots with their spline row, local coordinate and harmonics; the channel
// loops then run over the active slots only.  Spline rows are addressed
// through buffer resources built from wave-uniform (scalar) row bases, so a
// coefficient load costs no vector address arithmetic.
// ---------------------------------------------------------------------------
constexpr int kTile = 64;
static_assert(kTile == kEdgeTile, "edge-tile launches cut receivers at the kernels' tile size");

// The receiver and edge range of this workgroup: with an edge-tile list
// (LayerArgs::edge_tiles) one tile of at most edge_tile (<= kTile) edges,
// else all the receiver's edges.  `xcd` spreads consecutive entries over the XCDs in
// contiguous runs (receiver order); without it entry b is block b (the
// layer-0 type order).
__device__ __forceinline__ void block_edges(const LayerArgs& a, const int* tiles, bool xcd, int receiver, int& i,
                                            int& e0, int& e1)
{
    if (tiles) {
        const int b = xcd ? xcd_contiguous(blockIdx.x, a.num_edge_tiles) : static_cast<int>(blockIdx.x);
        i = tiles[2 * b];
        e0 = tiles[2 * b + 1];
        e1 = min(e0 + a.edge_tile, a.graph.first[i + 1]);
    } else {
        i = receiver;
        e0 = a.graph.first[i];
        e1 = a.graph.first[i + 1];
    }
}

// Streams the active slots 0..count-1 of a tile through a ring of D row
// buffers: the coefficient rows of the next D - 1 edges are in flight while
// one edge is processed.  fetch(j, buf) issues the loads of slot j into buf,
// use(j, buf) consumes them; all slot indices into the ring are compile-time.
template <int D, class Buf, class Fetch, class Use>
__device__ __forceinline__ void stream_ring(int count, Buf (&ring)[D], Fetch& fetch, Use& use)
{
#pragma unroll
    for (int d = 0; d < D - 1; ++d)
        if (d < count) fetch(d, ring[d]);
    for (int j = 0; j < count; j += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int jj = j + d;
            if (jj < count) {
                if (jj + D - 1 < count) fetch(jj + D - 1, ring[(d + D - 1) % D]);
                use(jj, ring[d]);
            }
        }
    }
}

constexpr int kDepth = 4;  // edges in flight per wave in the layer-0 kernels

// stream_ring (D = 4) for edge functions that yield three force components
// per lane: use(j, buf, f0, f1, f2).  The components of each group of four
// consecutive slots are summed over the wave together (wave_sum_3x4), and
// lane 16 r + 15 passes slot j + r's three sums to store(j + r, sums).
template <class Buf, class Fetch, class Use, class Store>
__device__ __forceinline__ void stream_ring_sum3(int count, Buf (&ring)[4], Fetch& fetch, Use& use, Store& store)
{
    constexpr int D = 4;
    const int r = (threadIdx.x & 63) >> 4;
    const bool holder = (threadIdx.x & 15) == 15;
#pragma unroll
    for (int d = 0; d < D - 1; ++d)
        if (d < count) fetch(d, ring[d]);
    for (int j = 0; j < count; j += D) {
        float f[3][D];
#pragma unroll
        for (int d = 0; d < D; ++d) f[0][d] = f[1][d] = f[2][d] = 0.0f;
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int jj = j + d;
            if (jj < count) {
                if (jj + D - 1 < count) fetch(jj + D - 1, ring[(d + D - 1) % D]);
                use(jj, ring[d], f[0][d], f[1][d], f[2][d]);
            }
        }
        float sums[3];
        wave_sum_3x4(f, sums);
        if (holder && j + r < count) store(j + r, sums);
    }
}

struct TileSlot {
    bool active;
    int slot;
    int row;  // spline coefficient row: pair * intervals + interval
    float x;  // local coordinate in the interval
};

// Compacts the edges [base, base + n) of the tile within r_cut into slots;
// lanes 0..63 of wave 0.  kOrdered selects the ordered-pair rows of the
// layer-0 tables, else the unordered (or shared) rows of the second
// interaction.  With kSorted the slots are ordered by spline row (ties in
// edge order): edges that share a coefficient row become neighbours in the
// channel loop and find the row in L1 (in a crystal most of a receiver's
// edges fall into a few shells); the slot is then the number of active lanes
// with a smaller (row, lane) key.  The forward kernels, bound by their row
// loads, sort; the reverse kernels, bound by arithmetic, keep edge order
// (slot = lane prefix count) and skip the ranking.
template <bool kOrdered, bool kSorted>
__device__ __forceinline__ TileSlot compact_edge(const EdgeGraph& g, const SplineGrid& grid, int base, int n,
                                                 int t, double& rr, int* count, bool pair_tables = false)
{
    bool on = false;
    rr = 0.0;
    int row = 0;
    float x = 0.0f;
    if (t < n) {
        rr = g.r[base + t - g.edge_base];
        on = rr < grid.r_cut;
    }
    if (on) {
        int iv;
        spline_point(rr, grid, iv, x);
        const int code = g.edge_pair[base + t - g.edge_base];
        // pair_tables: a layer-0 kernel on the unfolded table (rows per
        // unordered pair table, as the second interaction's)
        const int pair = kOrdered && !pair_tables ? code & 0xffff : code >> 16;
        row = pair * grid.intervals + iv;
    }
    const unsigned long long mask = __ballot(on);
    int slot;
    if constexpr (kSorted) {
        constexpr unsigned kRowCap = (1u << 26) - 2;  // keys stay below the inactive sentinel
        const unsigned key = on ? (min(static_cast<unsigned>(row), kRowCap) << 6) | static_cast<unsigned>(t)
                                : 0xffffffffu;
        slot = 0;
#pragma unroll
        for (int u = 0; u < 64; ++u)
            slot += static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(key), u)) < key ? 1 : 0;
    } else {
        slot = __builtin_amdgcn_mbcnt_hi(static_cast<unsigned>(mask >> 32),
                                         __builtin_amdgcn_mbcnt_lo(static_cast<unsigned>(mask), 0));
    }
    if (t == 0) *count = __popcll(mask);
    return {on, slot, row, x};
}

// Scalar density spline (one cubic per interval and unordered pair) at r:
// value and slope (reference CubicSpline evaluate / evaluate_deriv).
__device__ __forceinline__ float4v density_coef(const float* table, const SplineGrid& grid, int pair_u, double r,
                                                float& x)
{
    int iv;
    spline_point(r, grid, iv, x);
    return *reinterpret_cast<const float4v*>(table + 4 * (static_cast<size_t>(pair_u) * grid.intervals + iv));
}

__device__ __forceinline__ float density_value(const float* table, const SplineGrid& grid, int pair_u, double r)
{
    float x;
    const float4v c = density_coef(table, grid, pair_u, r, x);
    return cubic(c, x);
}

__device__ __forceinline__ float density_slope(const float* table, const SplineGrid& grid, int pair_u, double r)
{
    float x;
    const float4v c = density_coef(table, grid, pair_u, r, x);
    return cubic_slope(c, x, 3.0f * x);
}

// Sum over all edges [e0, e1) of the receiver of its density spline, by
// wave 0 (all 64 lanes), in a fixed order: returns 1 + sum on every lane.
__device__ __forceinline__ float density_scale(const DensityScale& d, const EdgeGraph& g, const SplineGrid& grid,
                                               int e0, int e1)
{
    float sum = 0.0f;
    for (int b = e0; b < e1; b += 64) {
        const int e = b + static_cast<int>(threadIdx.x);
        float v = 0.0f;
        if (e < e1) v = density_value(d.table, grid, g.edge_pair[e - g.edge_base] >> 16, g.r[e - g.edge_base]);
        sum += wave_sum_dpp(v);
    }
    return 1.0f + sum;
}

// ---------------------------------------------------------------------------
// Layer 0 forward: A0[i, lm, k] = sum_j R0f_{pair}(r_ij)[l, k] Y_lm(r_ij)
// ---------------------------------------------------------------------------
// kUnfolded: the table holds no H0 / A0_W (LayerArgs::h0); each edge's radial
// values are scaled by H0 of its source's type, A0 receives the sums before A0_W.
template <int LMAX, bool kUnfolded>
__global__ void __launch_bounds__(256) a0_forward_kernel(LayerArgs a, const float* __restrict__ r0f,
                                                          float* __restrict__ A0)
{
    constexpr int NLM = (LMAX + 1) * (LMAX + 1);
    constexpr int NL = LMAX + 1;
    __shared__ float s_Y[kTile][NLM];
    __shared__ float s_x[kTile];
    __shared__ int s_row[kTile];
    __shared__ int s_h0row[kTile];  // kUnfolded: offset of the source type's H0 row
    __shared__ int s_gstart[kTile + 1];  // first slot of each run of equal rows
    __shared__ int s_count, s_groups;

    __shared__ float s_scale;

    const int i = layer0_receiver(a);
    const int k = threadIdx.x;
    const int C = a.C;
    const EdgeGraph& g = a.graph;
    const int voff = min(k, C - 1) * 16;
    const int row_bytes = NL * C * 16;
    if (a.d0.table && threadIdx.x < 64) {
        const float sc = density_scale(a.d0, g, a.grid, g.first[i], g.first[i + 1]);
        if (threadIdx.x == 0) s_scale = sc;
    }
    float acc[NLM];
#pragma unroll
    for (int lm = 0; lm < NLM; ++lm) acc[lm] = 0.0f;
    const int e0 = g.first[i], e1 = g.first[i + 1];
    for (int base = e0; base < e1; base += kTile) {
        __syncthreads();
        if (threadIdx.x < 64) {
            const int t = threadIdx.x;
            double rr;
            const TileSlot ts =
                compact_edge<true, true>(g, a.grid, base, min(kTile, e1 - base), t, rr, &s_count, kUnfolded);
            if (ts.active) {
                const int e = base + t;
                float Y[NLM], dir[3];
                edge_harmonics<LMAX, false>(g.xyz + 3 * static_cast<size_t>(e - g.edge_base), rr, Y, nullptr,
                                            nullptr, nullptr, dir);
                s_x[ts.slot] = ts.x;
                s_row[ts.slot] = ts.row;
                if constexpr (kUnfolded)
                    s_h0row[ts.slot] = (g.edge_pair[e - g.edge_base] & 0xffff) % g.num_active * C;
#pragma unroll
                for (int lm = 0; lm < NLM; ++lm) s_Y[ts.slot][lm] = Y[lm];
            }
            // runs of equal rows among the (row-sorted) slots: lane t checks
            // slot t against slot t - 1
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const int count = uniform(s_count);
            const bool start = t < count && (t == 0 || s_row[t] != s_row[t - 1]);
            const unsigned long long starts = __ballot(start);
            const int g = __builtin_amdgcn_mbcnt_hi(static_cast<unsigned>(starts >> 32),
                                                    __builtin_amdgcn_mbcnt_lo(static_cast<unsigned>(starts), 0));
            if (start) s_gstart[g] = t;
            if (t == 0) {
                s_groups = __popcll(starts);
                s_gstart[__popcll(starts)] = count;
            }
        }
        __syncthreads();
        // one spline row per run of edges in the same interval, a ring of
        // kDepth rows in flight while earlier runs are accumulated
        const int groups = uniform(s_groups);
        auto fetch = [&](int gi, float4v* c) {
            const int row = uniform(s_row[uniform(s_gstart[gi])]);
            const auto rs = buffer_rsrc(r0f + static_cast<size_t>(row) * NL * C * 4, row_bytes);
#pragma unroll
            for (int l = 0; l < NL; ++l) c[l] = load4(rs, voff, l * C * 16);
        };
        auto accumulate = [&](int gi, const float4v* c) {
            const int j1 = uniform(s_gstart[gi + 1]);
            for (int j = uniform(s_gstart[gi]); j < j1; ++j) {
                const float x = uniform(s_x[j]);
                float R[NL];
#pragma unroll
                for (int l = 0; l < NL; ++l) R[l] = cubic(c[l], x);
                if constexpr (kUnfolded) {
                    const float h = a.h0[uniform(s_h0row[j]) + min(k, C - 1)];
#pragma unroll
                    for (int l = 0; l < NL; ++l) R[l] *= h;
                }
#pragma unroll
                for (int lm = 0; lm < NLM; ++lm) acc[lm] = fmaf(R[kLmL[lm]], s_Y[j][lm], acc[lm]);
            }
        };
        float4v ring[kDepth][NL];
        stream_ring<kDepth>(groups, ring, fetch, accumulate);
    }
    if (a.d0.table) {
        __syncthreads();
        const float sc = s_scale;
#pragma unroll
        for (int lm = 0; lm < NLM; ++lm) acc[lm] /= sc;
    }
    if (k < C) {
        float* out = A0 + static_cast<size_t>(i - a.local_base) * NLM * C + k;
#pragma unroll
        for (int lm = 0; lm < NLM; ++lm) out[lm * C] = acc[lm];
    }
}

// Channel-sliced layer-0 forward for graphs whose receivers leave SIMDs idle
// (LayerArgs::a0_slices = C / 64 workgroups per receiver): a workgroup runs
// one 64-channel slice of a receiver; each of its 4 waves takes a contiguous
// quarter of the receiver's edges and stages and consumes its own tiles of
// kWaveTile edges (sorted by spline row, one row load per run of equal rows,
// no workgroup barrier in the edge loop); the waves' partial sums are added
// at the end in a fixed order, (w0 + w2) + (w1 + w3).
template <int LMAX, bool kUnfolded>
__global__ void __launch_bounds__(256) a0_forward_sliced_kernel(LayerArgs a, const float* __restrict__ r0f,
                                                                 float* __restrict__ A0)
{
    constexpr int NLM = (LMAX + 1) * (LMAX + 1);
    constexpr int NL = LMAX + 1;
    constexpr int kWT = 16;  // edges per wave tile
    __shared__ float s_Y[kMaxWaves][kWT][NLM];
    __shared__ float s_x[kMaxWaves][kWT];
    __shared__ int s_row[kMaxWaves][kWT];
    __shared__ int s_h0row[kMaxWaves][kWT];
    __shared__ int s_gstart[kMaxWaves][kWT + 1];
    __shared__ int s_count[kMaxWaves], s_groups[kMaxWaves];
    __shared__ float s_red[2][NLM][64];
    __shared__ float s_scale;

    int slice;
    const int r = xcd_slice_receiver(blockIdx.x, a.node_count, a.a0_slices, slice);
    const int i = a.type_order ? a.type_order[a.node_offset + r] : a.node_offset + r;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int C = a.C;
    const int k = slice * 64 + lane;  // < C: C = 64 slices
    const EdgeGraph& g = a.graph;
    const int row_bytes = NL * C * 16;
    if (a.d0.table && wave == 0) {
        const float sc = density_scale(a.d0, g, a.grid, g.first[i], g.first[i + 1]);
        if (lane == 0) s_scale = sc;
    }
    float acc[NLM];
#pragma unroll
    for (int lm = 0; lm < NLM; ++lm) acc[lm] = 0.0f;
    const int e0 = g.first[i], n = g.first[i + 1] - e0;
    const int lo = e0 + (n * wave) / kMaxWaves, hi = e0 + (n * (wave + 1)) / kMaxWaves;
    for (int base = lo; base < hi; base += kWT) {
        // the wave's previous tile is consumed before its slots are rewritten
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        {
            double rr;
            const TileSlot ts = compact_edge<true, true>(g, a.grid, base, min(kWT, hi - base), lane, rr,
                                                         &s_count[wave], kUnfolded);
            if (ts.active) {
                const int e = base + lane;
                float Y[NLM], dir[3];
                edge_harmonics<LMAX, false>(g.xyz + 3 * static_cast<size_t>(e - g.edge_base), rr, Y, nullptr,
                                            nullptr, nullptr, dir);
                s_x[wave][ts.slot] = ts.x;
                s_row[wave][ts.slot] = ts.row;
                if constexpr (kUnfolded)
                    s_h0row[wave][ts.slot] = (g.edge_pair[e - g.edge_base] & 0xffff) % g.num_active * C;
#pragma unroll
                for (int lm = 0; lm < NLM; ++lm) s_Y[wave][ts.slot][lm] = Y[lm];
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            // runs of equal rows among the (row-sorted) slots
            const int count = uniform(s_count[wave]);
            const bool start = lane < count && (lane == 0 || s_row[wave][lane] != s_row[wave][lane - 1]);
            const unsigned long long starts = __ballot(start);
            const int gi = __builtin_amdgcn_mbcnt_hi(static_cast<unsigned>(starts >> 32),
                                                     __builtin_amdgcn_mbcnt_lo(static_cast<unsigned>(starts), 0));
            if (start) s_gstart[wave][gi] = lane;
            if (lane == 0) {
                s_groups[wave] = __popcll(starts);
                s_gstart[wave][__popcll(starts)] = count;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int groups = uniform(s_groups[wave]);
        auto fetch = [&](int gi, float4v* c) {
            const int row = uniform(s_row[wave][uniform(s_gstart[wave][gi])]);
            const auto rs = buffer_rsrc(r0f + static_cast<size_t>(row) * NL * C * 4, row_bytes);
#pragma unroll
            for (int l = 0; l < NL; ++l) c[l] = load4(rs, k * 16, l * C * 16);
        };
        auto accumulate = [&](int gi, const float4v* c) {
            const int j1 = uniform(s_gstart[wave][gi + 1]);
            for (int j = uniform(s_gstart[wave][gi]); j < j1; ++j) {
                const float x = uniform(s_x[wave][j]);
                float R[NL];
#pragma unroll
                for (int l = 0; l < NL; ++l) R[l] = cubic(c[l], x);
                if constexpr (kUnfolded) {
                    const float h = a.h0[uniform(s_h0row[wave][j]) + k];
#pragma unroll
                    for (int l = 0; l < NL; ++l) R[l] *= h;
                }
#pragma unroll
                for (int lm = 0; lm < NLM; ++lm) acc[lm] = fmaf(R[kLmL[lm]], s_Y[wave][j][lm], acc[lm]);
            }
        };
        float4v ring[kDepth][NL];
        stream_ring<kDepth>(groups, ring, fetch, accumulate);
    }
    __syncthreads();
    if (wave >= 2) {
#pragma unroll
        for (int lm = 0; lm < NLM; ++lm) s_red[wave - 2][lm][lane] = acc[lm];
    }
    __syncthreads();
    if (wave < 2) {
#pragma unroll
        for (int lm = 0; lm < NLM; ++lm) acc[lm] += s_red[wave][lm][lane];
    }
    __syncthreads();
    if (wave == 1) {
#pragma unroll
        for (int lm = 0; lm < NLM; ++lm) s_red[0][lm][lane] = acc[lm];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int lm = 0; lm < NLM; ++lm) acc[lm] += s_red[0][lm][lane];
        if (a.d0.table) {
            const float sc = s_scale;
#pragma unroll
            for (int lm = 0; lm < NLM; ++lm) acc[lm] /= sc;
        }
        float* out = A0 + static_cast<size_t>(i - a.local_base) * NLM * C + k;
#pragma unroll
        for (int lm = 0; lm < NLM; ++lm) out[lm * C] = acc[lm];
    }
}

// ---------------------------------------------------------------------------
// Layer 1 forward: Phi1[i, lme, k] = sum_j sum_t cg_t Y_{lm1_t} R1_{p_t}(r)[k] H1[src, lm2_t, k]
//
// The terms are grouped by (path, lm2, lme): the tile prologue folds each
// group's CG-weighted harmonics into one edge weight W_g = sum_t cg_t Y_lm1(t),
// and the channel loop does one FMA per group, acc[lme_g] += W_g R_p H_lm2.
// W is read from LDS in batches of kWBatch float4s, double-buffered, with
// scheduling barriers so each batch is in flight while the previous one is
// consumed (the compiler otherwise issues each read just before its use).
// ---------------------------------------------------------------------------
constexpr int kWBatch = 4;
// shapes with at most this many paths keep a spline row in registers for the
// next edge of the same interval
constexpr int kRowReusePaths = 10;

// The terms of a shape in the order of their edge-weight float4 (term_pl / 4):
// the staging loop visits each term once (an unrolled loop over all terms per
// float4 would be NT x NQ compile-time branches, too many to unroll for the
// wide shape).
template <class S>
struct R1TermsByQuad {
    static constexpr int NQ = (S::NPL + 3) / 4;
    int order[S::NT] = {};
    int start[NQ + 1] = {};
    constexpr R1TermsByQuad()
    {
        int n = 0;
        for (int q = 0; q < NQ; ++q) {
            start[q] = n;
            for (int u = 0; u < S::NT; ++u)
                if (S::term_pl[u] / 4 == q) order[n++] = u;
        }
        start[NQ] = n;
    }
};
template <class S>
inline constexpr R1TermsByQuad<S> kTermsByQuad{};

// Stages edge t of the tile [base, base + n) of a receiver's edges (lanes
// 0..63 of one wave): compacted slot, spline row, local coordinate, source
// and the folded edge weights W_g = sum_{t in g} cg_t Y_lm1(t) of the
// (path, lm2, lme) groups.
template <class S, bool kSorted>
__device__ __forceinline__ void r1_stage_edge(const LayerArgs& a, const float* __restrict__ cg, int base, int n,
                                              int t, float4v (*s_W)[(S::NPL + 3) / 4], float* s_x, int* s_row,
                                              int* s_src, int* s_count)
{
    constexpr int NLM = (S::LMAX + 1) * (S::LMAX + 1);
    constexpr int NQ = (S::NPL + 3) / 4;
    const EdgeGraph& g = a.graph;
    double rr;
    const TileSlot ts = compact_edge<false, kSorted>(g, a.grid, base, n, t, rr, s_count);
    if (ts.active) {
        const int e = base + t;
        float Y[NLM], dir[3];
        edge_harmonics<S::LMAX, false>(g.xyz + 3 * static_cast<size_t>(e - g.edge_base), rr, Y, nullptr, nullptr,
                                       nullptr, dir);
        s_x[ts.slot] = ts.x;
        s_row[ts.slot] = ts.row;
        s_src[ts.slot] = g.source[e];
        // one float4 of W at a time, over the terms of that float4
        constexpr const R1TermsByQuad<S>& tq = kTermsByQuad<S>;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            float4v w = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int v = tq.start[q]; v < tq.start[q + 1]; ++v) {
                const int u = tq.order[v];
                w[S::term_pl[u] % 4] = fmaf(cg[u], Y[S::term_lm1[u]], w[S::term_pl[u] % 4]);
            }
            s_W[ts.slot][q] = w;
        }
    }
}

// Channel loop over the staged slots [lo, hi) of a tile: per slot the radial
// values R_p(r) of the thread's channel kk (one coefficient row per slot,
// refilled for the next slot while this one is accumulated), the source
// features H1[src, lm2, kk], and acc[lme_g] += W_g R_p H_lm2 per group.
template <class S>
__device__ __forceinline__ void r1_forward_slots(const float4v (*s_W)[(S::NPL + 3) / 4], const float* s_x,
                                                 const int* s_row, const int* s_src, int lo, int hi, int C, int kk,
                                                 const float* __restrict__ r1, const float* __restrict__ H1,
                                                 float (&acc)[S::NLME])
{
    constexpr int NLMS = (S::LLMAX + 1) * (S::LLMAX + 1);
    constexpr int NP = S::NP;
    constexpr int NPQ = S::NPQ;
    constexpr int NPL = S::NPL;
    constexpr int NQ = (NPL + 3) / 4;                 // float4s of W per edge
    constexpr int NB = (NQ + kWBatch - 1) / kWBatch;  // batches per edge
    const int row_bytes = NP * C * 16;
    const int h_bytes = NLMS * C * 4;
    auto fetch_row = [&](int j, float4v* c) {
        const auto rs = buffer_rsrc(r1 + static_cast<size_t>(uniform(s_row[j])) * NP * C * 4, row_bytes);
#pragma unroll
        for (int p = 0; p < NP; ++p) c[p] = load4(rs, kk * 16, p * C * 16);
    };
    auto fetch_h = [&](int j, float* H) {
        const auto hs = buffer_rsrc(H1 + static_cast<size_t>(uniform(s_src[j])) * NLMS * C, h_bytes);
#pragma unroll
        for (int q = 0; q < NLMS; ++q) H[q] = load1(hs, kk * 4, q * C * 4);
    };
    // One row buffer: once the radial values of slot j are formed, its
    // coefficient registers are refilled with the row of slot j + 1 -- only
    // when that row differs: slots sorted by row let edges of one spline
    // interval reuse the registers (a wave-uniform branch; shapes with up to
    // kRowReusePaths paths).
    float4v c[NP];
    float H[NLMS];
    if (lo < hi) {
        fetch_row(lo, c);
        fetch_h(lo, H);
    }
    for (int j = lo; j < hi; ++j) {
        const float4v* Wj = s_W[j];
        float4v wb[2][kWBatch];
#pragma unroll
        for (int q = 0; q < kWBatch; ++q)
            if (q < NQ) wb[0][q] = Wj[q];
        const float x = uniform(s_x[j]);
        float RH[NPQ];
#pragma unroll
        for (int pq = 0; pq < NPQ; ++pq) RH[pq] = cubic(c[S::pq_p[pq]], x) * H[S::pq_lm2[pq]];
        if constexpr (S::NP <= kRowReusePaths) {
            // RH is formed here, before the conditional refill: left to the
            // compiler, the radial values sink below the branch, the refill
            // then needs a second row buffer and every edge pays a register
            // copy of the row at the loop latch
#pragma unroll
            for (int pq = 0; pq < NPQ; ++pq) asm volatile("" : : "v"(RH[pq]));
        }
        const int jn = min(j + 1, hi - 1);
        // (the wide shapes' row registers leave no room for the branch: they
        // reload, an L1 hit)
        if (S::NP > kRowReusePaths || uniform(s_row[jn]) != uniform(s_row[j])) fetch_row(jn, c);
        fetch_h(jn, H);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (b + 1 < NB) {
#pragma unroll
                for (int q = 0; q < kWBatch; ++q)
                    if ((b + 1) * kWBatch + q < NQ) wb[(b + 1) & 1][q] = Wj[(b + 1) * kWBatch + q];
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int q = 0; q < kWBatch; ++q) {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int gidx = 4 * (b * kWBatch + q) + u;
                    if (gidx < NPL)
                        acc[S::pl_lme[gidx]] = fmaf(wb[b & 1][q][u], RH[S::pl_pq[gidx]], acc[S::pl_lme[gidx]]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

template <class S>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(S::NPL <= 96 ? 3 : 1)))
r1_forward_kernel(LayerArgs a, const float* __restrict__ r1, const float* __restrict__ cg,
                  const float* __restrict__ H1, float* __restrict__ Phi1)
{
    constexpr int NQ = (S::NPL + 3) / 4;
    __shared__ float4v s_W[kTile][NQ];
    __shared__ float s_x[kTile];
    __shared__ int s_row[kTile];
    __shared__ int s_src[kTile];
    __shared__ int s_count;

    const int i = receiver_of_block(a);
    const int k = threadIdx.x;
    const int C = a.C;
    const EdgeGraph& g = a.graph;
    const int kk = min(k, C - 1);
    if (a.d1.table && threadIdx.x < 64) {
        const float sc = density_scale(a.d1, g, a.grid, g.first[i], g.first[i + 1]);
        if (threadIdx.x == 0) a.d1.scale[i] = sc;
    }
    float acc[S::NLME];
#pragma unroll
    for (int q = 0; q < S::NLME; ++q) acc[q] = 0.0f;
    const int e0 = g.first[i], e1 = g.first[i + 1];
    for (int base = e0; base < e1; base += kTile) {
        __syncthreads();
        if (threadIdx.x < 64)
            r1_stage_edge<S, true>(a, cg, base, min(kTile, e1 - base), threadIdx.x, s_W, s_x, s_row, s_src,
                                   &s_count);
        __syncthreads();
        r1_forward_slots<S>(s_W, s_x, s_row, s_src, 0, uniform(s_count), C, kk, r1, H1, acc);
    }
    if (k < C) {
        // Phi1 is written once and read once, by the A1 GEMM, after the whole
        // launch: non-temporal stores keep the L2s for the source rows and the
        // table (water: 7.18-7.20 -> 7.00-7.01 ms in an interleaved A/B)
        float* out = Phi1 + static_cast<size_t>(i - a.local_base) * S::NLME * C + k;
#pragma unroll
        for (int q = 0; q < S::NLME; ++q) __builtin_nontemporal_store(acc[q], &out[q * C]);
    }
}

// Channel-sliced forward (LayerArgs::channel_slices workgroups per receiver,
// XCD-aligned): a workgroup runs one 64-channel slice of a receiver; each of
// its 4 waves takes a contiguous quarter of the receiver's edges and stages
// and consumes its own tiles of kWaveTile edges (no workgroup barrier in the
// edge loop); the waves' partial sums are added at the end in a fixed order,
// (w0 + w2) + (w1 + w3), through the tiles' LDS.
constexpr int kWaveTile = 16;

template <class S>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(S::NPL <= 96 ? 3 : 1)))
r1_forward_sliced_kernel(LayerArgs a, const float* __restrict__ r1, const float* __restrict__ cg,
                         const float* __restrict__ H1, float* __restrict__ Phi1)
{
    constexpr int NQ = (S::NPL + 3) / 4;
    __shared__ float4v s_W[kMaxWaves][kWaveTile][NQ];
    __shared__ float s_x[kMaxWaves][kWaveTile];
    __shared__ int s_row[kMaxWaves][kWaveTile];
    __shared__ int s_src[kMaxWaves][kWaveTile];
    __shared__ int s_count[kMaxWaves];

    int slice;
    const int i = a.node_offset + xcd_slice_receiver(blockIdx.x, a.node_count, a.channel_slices, slice);
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int C = a.C;
    const int k = slice * 64 + lane;  // < C: C = 64 slices
    const EdgeGraph& g = a.graph;
    if (a.d1.table && wave == 0) {
        const float sc = density_scale(a.d1, g, a.grid, g.first[i], g.first[i + 1]);
        if (lane == 0 && slice == 0) a.d1.scale[i] = sc;
    }
    float acc[S::NLME];
#pragma unroll
    for (int q = 0; q < S::NLME; ++q) acc[q] = 0.0f;
    const int e0 = g.first[i], n = g.first[i + 1] - e0;
    const int lo = e0 + (n * wave) / kMaxWaves, hi = e0 + (n * (wave + 1)) / kMaxWaves;
    for (int base = lo; base < hi; base += kWaveTile) {
        // the wave's previous tile is consumed before its slots are rewritten
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        r1_stage_edge<S, (S::NP <= kRowReusePaths)>(a, cg, base, min(kWaveTile, hi - base), lane, s_W[wave],
                                                     s_x[wave], s_row[wave], s_src[wave], &s_count[wave]);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        r1_forward_slots<S>(s_W[wave], s_x[wave], s_row[wave], s_src[wave], 0, uniform(s_count[wave]), C, k, r1,
                            H1, acc);
    }
    // partial sums of the 4 waves, kRows rows of the receiver's Phi1 at a time
    float* red = reinterpret_cast<float*>(&s_W[0][0][0]);
    constexpr int kCap = kMaxWaves * kWaveTile * NQ * 4 / 128;
    constexpr int kRows = kCap < S::NLME ? kCap : S::NLME;
#pragma unroll
    for (int r0 = 0; r0 < S::NLME; r0 += kRows) {
        __syncthreads();
        if (wave >= 2) {
#pragma unroll
            for (int q = 0; q < S::NLME; ++q)
                if (q >= r0 && q < r0 + kRows) red[((wave - 2) * kRows + q - r0) * 64 + lane] = acc[q];
        }
        __syncthreads();
        if (wave < 2) {
#pragma unroll
            for (int q = 0; q < S::NLME; ++q)
                if (q >= r0 && q < r0 + kRows) acc[q] += red[(wave * kRows + q - r0) * 64 + lane];
        }
        __syncthreads();
        if (wave == 1) {
#pragma unroll
            for (int q = 0; q < S::NLME; ++q)
                if (q >= r0 && q < r0 + kRows) red[(q - r0) * 64 + lane] = acc[q];
        }
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int q = 0; q < S::NLME; ++q)
                if (q >= r0 && q < r0 + kRows) acc[q] += red[(q - r0) * 64 + lane];
        }
    }
    if (wave == 0) {
        float* out = Phi1 + static_cast<size_t>(i - a.local_base) * S::NLME * C + k;
#pragma unroll
        for (int q = 0; q < S::NLME; ++q) __builtin_nontemporal_store(acc[q], &out[q * C]);
    }
}

// The (path, lm2, lm1) triples of a shape or path group are contiguous per
// (path, lm2) pair (term order): start[pq] .. start[pq + 1].
template <class RG>
struct RevTrRanges {
    int start[RG::NPQ + 1] = {};
    bool ordered = true;
    constexpr RevTrRanges()
    {
        int pq = 0;
        for (int tr = 0; tr < RG::NTR; ++tr) {
            if (RG::tr_pq[tr] < pq) ordered = false;
            while (pq < RG::tr_pq[tr]) start[++pq] = tr;
        }
        while (pq < RG::NPQ) start[++pq] = RG::NTR;
    }
};
template <class RG>
inline constexpr RevTrRanges<RG> kRevTrRanges{};

// The harmonic part of a layer-1 edge force, g = sum_lm U_lm dY_lm/dr, is
// tangential: Y_lm depends on the direction r_hat only, so r_hat . dY_lm/dr
// = 0 for every lm.  Two Cartesian components therefore fix g.  The staging
// keeps the gradient rows of the two axes other than `drop`, the axis where
// |r_hat| is largest (|r_hat_drop| >= 1/sqrt(3)); the channels reduce only
// those two components; the edge's thread forms the third as
// -(r_a g_a + r_b g_b) / r_drop.  Rows of l = 0 are zero and left out: a
// staged row holds lm = 1 .. NLM - 1 at index lm - 1 (16-byte aligned reads).
template <int NLM>
__device__ __forceinline__ void stage_tangent_rows(const float (&dY)[3][NLM], const float* u, float* row_a,
                                                   float* row_b, int& drop)
{
    const float ax = fabsf(u[0]), ay = fabsf(u[1]), az = fabsf(u[2]);
    drop = (az >= ax && az >= ay) ? 2 : (ay >= ax ? 1 : 0);
#pragma unroll
    for (int lm = 1; lm < NLM; ++lm) {
        row_a[lm - 1] = drop == 0 ? dY[1][lm] : dY[0][lm];
        row_b[lm - 1] = drop == 2 ? dY[1][lm] : dY[2][lm];
    }
}

// +dE/dr of an edge from the channel sums of the radial coefficient A and of
// the two kept harmonic components (ga on the lower kept axis, gb on the upper).
__device__ __forceinline__ void tangent_force(double A, double ga, double gb, int drop, const float* u,
                                              double (&f)[3])
{
    const double ux = u[0], uy = u[1], uz = u[2];
    const double ua = drop == 0 ? uy : ux;
    const double ub = drop == 2 ? uy : uz;
    const double ud = drop == 0 ? ux : (drop == 1 ? uy : uz);
    const double gd = -(ua * ga + ub * gb) / ud;
    f[0] = fma(ux, A, drop == 0 ? gd : ga);
    f[1] = fma(uy, A, drop == 0 ? ga : (drop == 1 ? gd : gb));
    f[2] = fma(uz, A, drop == 2 ? gd : gb);
}

// ---------------------------------------------------------------------------
// Layer 1 reverse.  Per receiver and channel, the CG contraction of dPhi1 is
// taken once: G[p, lm2, lm1] = sum_{t in (p, lm2, lm1)} cg_t dPhi1[lme_t].
// Per edge:
//   s[p,lm2]  = sum_lm1 Y_lm1 G[p,lm2,lm1]
//   msg[lm2]  = sum_p R_p s[p,lm2]                   -> H1 adjoint of the source
//   A         = sum_p R'_p sum_lm2 H[lm2] s[p,lm2]
//   U[lm1]    = sum_{p,lm2} R_p H[lm2] G[p,lm2,lm1]
//   f_edge    = -(r_hat A + sum_lm1 dY[lm1] U[lm1])
// with the harmonic term reduced as two tangential components
// (stage_tangent_rows).  When G does not fit the register budget (many
// triples) the terms are contracted per edge instead, with dPhi1 in
// registers.
// ---------------------------------------------------------------------------
template <class S>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(S::NTR <= 40 ? 3 : 1)))
r1_reverse_kernel(LayerArgs a, const float* __restrict__ r1,
                                                         const float* __restrict__ cg,
                                                         const float* __restrict__ H1,
                                                         const float* __restrict__ dPhi1,
                                                         double* __restrict__ forces,
                                                         float* __restrict__ msg)
{
    constexpr int NLM = (S::LMAX + 1) * (S::LMAX + 1);
    constexpr int NLMS = (S::LLMAX + 1) * (S::LLMAX + 1);
    constexpr int NP = S::NP;
    constexpr int NT = S::NT;
    constexpr int NPQ = S::NPQ;
    constexpr bool kFactored = S::NTR <= 96;
    constexpr int NG = kFactored ? S::NTR : S::NLME;
    constexpr int NCGY = kFactored ? 1 : (NT + 3) / 4 * 4;
    __shared__ float s_Y[kTile][NLM];
    __shared__ float s_dT[kTile][2][(NLM + 2) / 4 * 4];  // the two kept gradient rows (stage_tangent_rows)
    __shared__ int s_drop[kTile];
    __shared__ float s_geo[kTile][4];  // r_hat, local spline coordinate
    __shared__ float s_cgY[kTile][NCGY];
    __shared__ int s_row[kTile];
    __shared__ int s_src[kTile];
    __shared__ int s_eid[kTile];
    __shared__ float s_f[kTile][kMaxWaves * kForceParts][3];
    __shared__ float s_dsc[kTile];  // A1 density-scale force coefficient per active slot
    __shared__ int s_count;

    int i, e0, e1;
    block_edges(a, a.edge_tiles, true, a.edge_tiles ? 0 : receiver_of_block(a), i, e0, e1);
    const int k = threadIdx.x;
    const int C = a.C;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int nwaves = blockDim.x >> 6;
    const EdgeGraph& g = a.graph;
    const int kk = min(k, C - 1);
    const int row_bytes = NP * C * 16;
    const int h_bytes = NLMS * C * 4;
    // (A1_adj . A1) / s of this receiver (reverse_A1_scaled)
    const float dcoef = a.d1.table ? a.d1.dot[i] / a.d1.scale[i] : 0.0f;
    // G (factored) or dPhi1 (per-term); zero on lanes beyond C
    float G[NG];
#pragma unroll
    for (int q = 0; q < NG; ++q) G[q] = 0.0f;
    if (k < C) {
        const float* in = dPhi1 + static_cast<size_t>(i - a.local_base) * S::NLME * C + k;
        if constexpr (kFactored) {
            float d[S::NLME];
#pragma unroll
            for (int q = 0; q < S::NLME; ++q) d[q] = in[q * C];
#pragma unroll
            for (int t = 0; t < NT; ++t) G[S::term_tr[t]] = fmaf(cg[t], d[S::term_lme[t]], G[S::term_tr[t]]);
        } else {
#pragma unroll
            for (int q = 0; q < S::NLME; ++q) G[q] = in[q * C];
        }
    }
    for (int base = e0; base < e1; base += kTile) {
        __syncthreads();
        if (threadIdx.x < 64) {
            const int t = threadIdx.x;
            double rr;
            const int n = min(kTile, e1 - base);
            const TileSlot ts = compact_edge<false, false>(g, a.grid, base, n, t, rr, &s_count);
            const int e = base + t;
            if (ts.active) {
                const int sl = ts.slot;
                float dY[3][NLM], u[3];
                edge_harmonics<S::LMAX, true>(g.xyz + 3 * static_cast<size_t>(e - g.edge_base), rr, s_Y[sl], dY[0],
                                              dY[1], dY[2], u);
                stage_tangent_rows<NLM>(dY, u, s_dT[sl][0], s_dT[sl][1], s_drop[sl]);
                s_geo[sl][0] = u[0];
                s_geo[sl][1] = u[1];
                s_geo[sl][2] = u[2];
                s_geo[sl][3] = ts.x;
                s_row[sl] = ts.row;
                s_src[sl] = g.source[e];
                s_eid[sl] = e;
                s_dsc[sl] = a.d1.table ? dcoef * density_slope(a.d1.table, a.grid, g.edge_pair[e - g.edge_base] >> 16, rr) : 0.0f;
                if constexpr (!kFactored) {
#pragma unroll
                    for (int q = 0; q < NT; ++q) s_cgY[sl][q] = cg[q] * s_Y[sl][S::term_lm1[q]];
                }
            } else if (t < n) {
                // beyond r_cut: only the A1 density-scale term (reverse_A1_scaled visits every neighbour)
                double* out = forces + 3 * static_cast<size_t>(e - g.edge_base);
                float d = 0.0f;
                if (a.d1.table) d = dcoef * density_slope(a.d1.table, a.grid, g.edge_pair[e - g.edge_base] >> 16, rr);
                const double* x = g.xyz + 3 * static_cast<size_t>(e - g.edge_base);
                out[0] = static_cast<double>(d * static_cast<float>(x[0] / rr));
                out[1] = static_cast<double>(d * static_cast<float>(x[1] / rr));
                out[2] = static_cast<double>(d * static_cast<float>(x[2] / rr));
            }
        }
        __syncthreads();
        const int count = uniform(s_count);
        auto fetch = [&](int j, float4v* c, float* H) {
            const auto rs = buffer_rsrc(r1 + static_cast<size_t>(uniform(s_row[j])) * NP * C * 4, row_bytes);
            const auto hs = buffer_rsrc(H1 + static_cast<size_t>(uniform(s_src[j])) * NLMS * C, h_bytes);
#pragma unroll
            for (int p = 0; p < NP; ++p) c[p] = load4(rs, kk * 16, p * C * 16);
#pragma unroll
            for (int q = 0; q < NLMS; ++q) H[q] = load1(hs, kk * 4, q * C * 4);
        };
        // One row buffer: once the radial values of edge j are formed, its
        // coefficient registers are refilled with the row of edge j + 1.
        // edge j from its row buffer (cj, Hj); the row of edge j + 1 is
        // already in flight in the other buffer
        auto edge = [&](int j, const float4v* cj, const float* Hj) {
            const float x = uniform(s_geo[j][3]);
            float R[NP], dR[NP], H[NLMS];
#pragma unroll
            for (int p = 0; p < NP; ++p) cubic_value_slope(cj[p], x, R[p], dR[p]);
#pragma unroll
            for (int q = 0; q < NLMS; ++q) H[q] = Hj[q];
            float sp[NPQ], U[NLM], RH[NPQ];
#pragma unroll
            for (int pq = 0; pq < NPQ; ++pq) {
                sp[pq] = 0.0f;
                RH[pq] = R[S::pq_p[pq]] * H[S::pq_lm2[pq]];
            }
#pragma unroll
            for (int lm = 0; lm < NLM; ++lm) U[lm] = 0.0f;
            if constexpr (kFactored) {
#pragma unroll
                for (int tr = 0; tr < S::NTR; ++tr) {
                    sp[S::tr_pq[tr]] = fmaf(s_Y[j][S::tr_lm1[tr]], G[tr], sp[S::tr_pq[tr]]);
                    U[S::tr_lm1[tr]] = fmaf(RH[S::tr_pq[tr]], G[tr], U[S::tr_lm1[tr]]);
                }
            } else {
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const int pq = S::tr_pq[S::term_tr[t]];
                    const float d = G[S::term_lme[t]];
                    sp[pq] = fmaf(s_cgY[j][t], d, sp[pq]);
                    U[S::term_lm1[t]] = fmaf(cg[t], RH[pq] * d, U[S::term_lm1[t]]);
                }
            }
            float m[NLMS], ap[NP];
#pragma unroll
            for (int q = 0; q < NLMS; ++q) m[q] = 0.0f;
#pragma unroll
            for (int p = 0; p < NP; ++p) ap[p] = 0.0f;
#pragma unroll
            for (int pq = 0; pq < NPQ; ++pq) {
                m[S::pq_lm2[pq]] = fmaf(R[S::pq_p[pq]], sp[pq], m[S::pq_lm2[pq]]);
                ap[S::pq_p[pq]] = fmaf(H[S::pq_lm2[pq]], sp[pq], ap[S::pq_p[pq]]);
            }
            float A = 0.0f;
#pragma unroll
            for (int p = 0; p < NP; ++p) A = fmaf(dR[p], ap[p], A);
            const int e = uniform(s_eid[j]);
            if (k < C) {
                const auto ms = buffer_rsrc(msg + static_cast<size_t>(e - a.graph.edge_base) * NLMS * C, h_bytes);
#pragma unroll
                for (int q = 0; q < NLMS; ++q) store1_stream(m[q], ms, k * 4, q * C * 4);
            }
            float ga = 0.0f, gb = 0.0f;
#pragma unroll
            for (int lm = 1; lm < NLM; ++lm) {
                ga = fmaf(s_dT[j][0][lm - 1], U[lm], ga);
                gb = fmaf(s_dT[j][1][lm - 1], U[lm], gb);
            }
            // partial sums of A and of the two kept harmonic components
            const float pA = partial_sum_dpp<kForceParts>(A);
            const float pa = partial_sum_dpp<kForceParts>(ga);
            const float pb = partial_sum_dpp<kForceParts>(gb);
            if (holds_partial<kForceParts>(lane)) {
                const int part = wave * kForceParts + lane / (64 / kForceParts);
                s_f[j][part][0] = pA;
                s_f[j][part][1] = pa;
                s_f[j][part][2] = pb;
            }
        };
        // Two row buffers used in turn (unrolled by two, so no register
        // copies).
        // A pair loop plus a one-edge tail keeps every path into the loop
        // head alike (a conditional second half would make the compiler wait
        // for the prefetch there).
        float4v ca[NP], cb[NP];
        float Ha[NLMS], Hb[NLMS];
        if (count > 0) fetch(0, ca, Ha);
        for (int j = 0; j + 1 < count; j += 2) {
            fetch(j + 1, cb, Hb);
            edge(j, ca, Ha);
            fetch(min(j + 2, count - 1), ca, Ha);
            edge(j + 1, cb, Hb);
        }
        if (count & 1) edge(count - 1, ca, Ha);
        __syncthreads();
        if (threadIdx.x < count) {
            const int t = threadIdx.x;
            double p[3] = {0.0, 0.0, 0.0};
            for (int w = 0; w < nwaves * kForceParts; ++w)
                for (int c = 0; c < 3; ++c) p[c] += static_cast<double>(s_f[t][w][c]);
            double f[3];
            tangent_force(p[0], p[1], p[2], s_drop[t], s_geo[t], f);
            double* out = forces + 3 * static_cast<size_t>(s_eid[t] - g.edge_base);
#pragma unroll
            for (int c = 0; c < 3; ++c) out[c] = -f[c] + static_cast<double>(s_dsc[t] * s_geo[t][c]);
        }
    }
}
// ---------------------------------------------------------------------------
// Layer 1 reverse in path-group passes, for shapes whose per-channel state
// does not fit one thread's registers in a single pass (R1Groups): per edge
// tile, pass G handles the paths of its source-l2 group, writes those message
// rows complete and adds its part of each edge force (the force is linear in
// the per-path terms).  The tile's edge geometry is staged once for all
// passes.
// ---------------------------------------------------------------------------
template <class S, int G>
using RevGroup = R1RevGroup<S::LMAX, S::LLMAX, G>;

template <int MAXT, int NPART = kMaxWaves * kForcePartsGrouped>
struct alignas(16) RevTileLds {
    float Y[kTile][16];
    float dT[kTile][2][16];  // the two kept gradient rows (stage_tangent_rows)
    int drop[kTile];
    float geo[kTile][4];  // r_hat, local spline coordinate
    float cgY[kTile][MAXT];
    int row[kTile];
    int src[kTile];
    int eid[kTile];
    float f[kTile][NPART][3];
    float dsc[kTile];
    int count;
};


// Channel k of this thread; the wave's force partials go to L.f[.][part0 ..].
template <class S, class RG, int MAXT, int NPART>
__device__ __forceinline__ void r1_reverse_pass(const LayerArgs& a, int i, bool first, int count, int k, int part0,
                                                const float* __restrict__ r1, const float* __restrict__ cg,
                                                const float* __restrict__ H1, const float* __restrict__ dPhi1,
                                                float* __restrict__ msg, RevTileLds<MAXT, NPART>& L)
{
    constexpr int NLM = (S::LMAX + 1) * (S::LMAX + 1);
    constexpr int NLMS = (S::LLMAX + 1) * (S::LLMAX + 1);
    constexpr int NG = RG::FACTORED ? RG::NTR : RG::NROW;
    const int C = a.C;
    const int lane = threadIdx.x & 63;
    const int kk = min(k, C - 1);
    const int row_bytes = S::NP * C * 16;
    const int h_bytes = NLMS * C * 4;
    // this group's dPhi1 rows, contracted with the CG coefficients per
    // (path, lm2, lm1) triple when the triples fit the register budget.  They
    // are reloaded per tile (an opaque zero offset keeps the compiler from
    // hoisting every pass's rows out of the tile loop at once).
    float G[NG];
#pragma unroll
    for (int q = 0; q < NG; ++q) G[q] = 0.0f;
    if (k < C) {
        int zero;
        asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
        const float* in = dPhi1 + static_cast<size_t>(i - a.local_base) * S::NLME * C + k + zero;
        if constexpr (RG::FACTORED) {
            float d[RG::NROW];
#pragma unroll
            for (int q = 0; q < RG::NROW; ++q) d[q] = in[RG::row_lme[q] * C];
#pragma unroll
            for (int t = 0; t < RG::NT; ++t)
                G[RG::term_tr[t]] = fmaf(cg[RG::term[t]], d[RG::term_row[t]], G[RG::term_tr[t]]);
        } else {
#pragma unroll
            for (int q = 0; q < RG::NROW; ++q) G[q] = in[RG::row_lme[q] * C];
        }
    }
    if constexpr (!RG::FACTORED) {
        __syncthreads();  // the previous pass has finished reading cgY
        if (threadIdx.x < count) {
            const int j = threadIdx.x;
#pragma unroll
            for (int t = 0; t < RG::NT; ++t) L.cgY[j][t] = cg[RG::term[t]] * L.Y[j][RG::term_lm1[t]];
        }
        __syncthreads();
    }
    auto fetch = [&](int j, float4v* c, float* H) {
        const auto rs = buffer_rsrc(r1 + static_cast<size_t>(uniform(L.row[j])) * S::NP * C * 4, row_bytes);
        const auto hs = buffer_rsrc(H1 + static_cast<size_t>(uniform(L.src[j])) * NLMS * C, h_bytes);
#pragma unroll
        for (int p = 0; p < RG::NP; ++p) c[p] = load4(rs, kk * 16, RG::path[p] * C * 16);
#pragma unroll
        for (int q = 0; q < RG::NH; ++q) H[q] = load1(hs, kk * 4, RG::h_lm2[q] * C * 4);
    };
    float4v cn[RG::NP];
    float Hn[RG::NH];
    if (count > 0) fetch(0, cn, Hn);
    for (int j = 0; j < count; ++j) {
        const float x = uniform(L.geo[j][3]);
        float R[RG::NP], dR[RG::NP], H[RG::NH];
#pragma unroll
        for (int p = 0; p < RG::NP; ++p) cubic_value_slope(cn[p], x, R[p], dR[p]);
#pragma unroll
        for (int q = 0; q < RG::NH; ++q) H[q] = Hn[q];
        fetch(min(j + 1, count - 1), cn, Hn);
        float U[NLM], m[RG::NH], ap[RG::NP];
#pragma unroll
        for (int lm = 0; lm < NLM; ++lm) U[lm] = 0.0f;
#pragma unroll
        for (int q = 0; q < RG::NH; ++q) m[q] = 0.0f;
#pragma unroll
        for (int p = 0; p < RG::NP; ++p) ap[p] = 0.0f;
        if constexpr (RG::FACTORED) {
            static_assert(kRevTrRanges<RG>.ordered, "triples of a (path, lm2) pair are not contiguous");
            // one (path, lm2) pair at a time: its triples' sum sp is consumed
            // at once, so no per-pair arrays are held
            constexpr const RevTrRanges<RG>& tq = kRevTrRanges<RG>;
            float Y[NLM];
#pragma unroll
            for (int lm = 0; lm < NLM; ++lm) Y[lm] = L.Y[j][lm];
#pragma unroll
            for (int pq = 0; pq < RG::NPQ; ++pq) {
                const int p = RG::pq_p[pq], h = RG::pq_h[pq];
                const float rh = R[p] * H[h];
                float sp = 0.0f;
#pragma unroll
                for (int tr = tq.start[pq]; tr < tq.start[pq + 1]; ++tr) {
                    sp = fmaf(Y[RG::tr_lm1[tr]], G[tr], sp);
                    U[RG::tr_lm1[tr]] = fmaf(rh, G[tr], U[RG::tr_lm1[tr]]);
                }
                m[h] = fmaf(R[p], sp, m[h]);
                ap[p] = fmaf(H[h], sp, ap[p]);
            }
        } else {
            float sp[RG::NPQ], RH[RG::NPQ];
#pragma unroll
            for (int pq = 0; pq < RG::NPQ; ++pq) {
                sp[pq] = 0.0f;
                RH[pq] = R[RG::pq_p[pq]] * H[RG::pq_h[pq]];
            }
#pragma unroll
            for (int t = 0; t < RG::NT; ++t) {
                const int pq = RG::tr_pq[RG::term_tr[t]];
                const float d = G[RG::term_row[t]];
                sp[pq] = fmaf(L.cgY[j][t], d, sp[pq]);
                U[RG::term_lm1[t]] = fmaf(cg[RG::term[t]], RH[pq] * d, U[RG::term_lm1[t]]);
            }
#pragma unroll
            for (int pq = 0; pq < RG::NPQ; ++pq) {
                m[RG::pq_h[pq]] = fmaf(R[RG::pq_p[pq]], sp[pq], m[RG::pq_h[pq]]);
                ap[RG::pq_p[pq]] = fmaf(H[RG::pq_h[pq]], sp[pq], ap[RG::pq_p[pq]]);
            }
        }
        float A = 0.0f;
#pragma unroll
        for (int p = 0; p < RG::NP; ++p) A = fmaf(dR[p], ap[p], A);
        const int e = uniform(L.eid[j]);
        if (k < C) {
            const auto ms = buffer_rsrc(msg + static_cast<size_t>(e - a.graph.edge_base) * NLMS * C, h_bytes);
#pragma unroll
            for (int q = 0; q < RG::NH; ++q) store1_stream(m[q], ms, k * 4, RG::h_lm2[q] * C * 4);
        }
        float ga = 0.0f, gb = 0.0f;
#pragma unroll
        for (int lm = 1; lm < NLM; ++lm) {
            ga = fmaf(L.dT[j][0][lm - 1], U[lm], ga);
            gb = fmaf(L.dT[j][1][lm - 1], U[lm], gb);
        }
        // partial sums of A and of the two kept harmonic components
        const float pA = partial_sum_dpp<kForcePartsGrouped>(A);
        const float pa = partial_sum_dpp<kForcePartsGrouped>(ga);
        const float pb = partial_sum_dpp<kForcePartsGrouped>(gb);
        if (holds_partial<kForcePartsGrouped>(lane)) {
            const int part = part0 + lane / (64 / kForcePartsGrouped);
            L.f[j][part][0] = first ? pA : L.f[j][part][0] + pA;
            L.f[j][part][1] = first ? pa : L.f[j][part][1] + pa;
            L.f[j][part][2] = first ? pb : L.f[j][part][2] + pb;
        }
    }
}

template <class S, int... G>
constexpr int rev_group_terms()
{
    int m = 1;
    ((m = !RevGroup<S, G>::FACTORED && RevGroup<S, G>::NT > m ? RevGroup<S, G>::NT : m), ...);
    return (m + 3) / 4 * 4;
}

// Wave 0 stages a tile of up to 64 of receiver i's edges from `base` for the
// path-group passes; an edge beyond r_cut gets only the A1 density-scale
// force term (reverse_A1_scaled visits every neighbour), passed to
// out(edge, term) with term = 0 when the model has no A1 density scale.
template <class S, int MAXT, int NPART, class Out>
__device__ __forceinline__ void stage_reverse_tile(const LayerArgs& a, int base, int e1, float dcoef,
                                                   RevTileLds<MAXT, NPART>& L, Out out)
{
    const EdgeGraph& g = a.graph;
    const int t = threadIdx.x;
    double rr;
    const int n = min(kTile, e1 - base);
    const TileSlot ts = compact_edge<false, false>(g, a.grid, base, n, t, rr, &L.count);
    const int e = base + t;
    if (ts.active) {
        const int sl = ts.slot;
        constexpr int NLM = (S::LMAX + 1) * (S::LMAX + 1);
        float dY[3][NLM], u[3];
        edge_harmonics<S::LMAX, true>(g.xyz + 3 * static_cast<size_t>(e - g.edge_base), rr, L.Y[sl], dY[0], dY[1],
                                      dY[2], u);
        stage_tangent_rows<NLM>(dY, u, L.dT[sl][0], L.dT[sl][1], L.drop[sl]);
        L.geo[sl][0] = u[0];
        L.geo[sl][1] = u[1];
        L.geo[sl][2] = u[2];
        L.geo[sl][3] = ts.x;
        L.row[sl] = ts.row;
        L.src[sl] = g.source[e];
        L.eid[sl] = e;
        L.dsc[sl] =
            a.d1.table ? dcoef * density_slope(a.d1.table, a.grid, g.edge_pair[e - g.edge_base] >> 16, rr) : 0.0f;
    } else if (t < n) {
        float d = 0.0f;
        if (a.d1.table) d = dcoef * density_slope(a.d1.table, a.grid, g.edge_pair[e - g.edge_base] >> 16, rr);
        out(e, d, rr);
    }
}

template <class S, int... G>
__global__ void __launch_bounds__(256) r1_reverse_grouped_kernel(LayerArgs a, const float* __restrict__ r1,
                                                                  const float* __restrict__ cg,
                                                                  const float* __restrict__ H1,
                                                                  const float* __restrict__ dPhi1,
                                                                  double* __restrict__ forces,
                                                                  float* __restrict__ msg)
{
    constexpr int MAXT = rev_group_terms<S, G...>();
    static_assert((S::LMAX + 1) * (S::LMAX + 1) <= 16, "harmonics beyond l = 3");
    __shared__ RevTileLds<MAXT> L;
    const int i = receiver_of_block(a);
    const int nwaves = blockDim.x >> 6;
    const EdgeGraph& g = a.graph;
    const float dcoef = a.d1.table ? a.d1.dot[i] / a.d1.scale[i] : 0.0f;
    const int e0 = g.first[i], e1 = g.first[i + 1];
    for (int base = e0; base < e1; base += kTile) {
        __syncthreads();
        if (threadIdx.x < 64)
            stage_reverse_tile<S>(a, base, e1, dcoef, L, [&](int e, float d, double rr) {
                double* out = forces + 3 * static_cast<size_t>(e - g.edge_base);
                const double* x = g.xyz + 3 * static_cast<size_t>(e - g.edge_base);
#pragma unroll
                for (int c = 0; c < 3; ++c) out[c] = static_cast<double>(d * static_cast<float>(x[c] / rr));
            });
        __syncthreads();
        const int count = uniform(L.count);
        (r1_reverse_pass<S, RevGroup<S, G>>(a, i, G == 0, count, threadIdx.x, (threadIdx.x >> 6) * kForcePartsGrouped,
                                            r1, cg, H1, dPhi1, msg, L),
         ...);
        __syncthreads();
        if (threadIdx.x < count) {
            const int t = threadIdx.x;
            double p[3] = {0.0, 0.0, 0.0};
            for (int w = 0; w < nwaves * kForcePartsGrouped; ++w)
                for (int c = 0; c < 3; ++c) p[c] += static_cast<double>(L.f[t][w][c]);
            double f[3];
            tangent_force(p[0], p[1], p[2], L.drop[t], L.geo[t], f);
            double* out = forces + 3 * static_cast<size_t>(L.eid[t] - g.edge_base);
#pragma unroll
            for (int c = 0; c < 3; ++c) out[c] = -f[c] + static_cast<double>(L.dsc[t] * L.geo[t][c]);
        }
    }
}

// Channel-sliced reverse (LayerArgs::channel_slices workgroups per receiver,
// XCD-aligned like the sliced forward): a one-wave workgroup runs the
// path-group passes of one 64-channel slice of a receiver, so each XCD's L2
// holds only its slice's columns of the coefficient table.  The slice's part
// of each directed force, a sum over its channels, goes to
// part[edge][slice][3] (slice 0 adds the A1 density-scale term, the other
// slices write zero for edges beyond r_cut); fold_slices_kernel adds the
// parts in slice order.
template <class S, int... G>
__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2)))
r1_reverse_sliced_kernel(LayerArgs a, const float* __restrict__ r1, const float* __restrict__ cg,
                         const float* __restrict__ H1, const float* __restrict__ dPhi1, double* __restrict__ part,
                         float* __restrict__ msg)
{
    constexpr int MAXT = rev_group_terms<S, G...>();
    static_assert((S::LMAX + 1) * (S::LMAX + 1) <= 16, "harmonics beyond l = 3");
    __shared__ RevTileLds<MAXT, kForcePartsGrouped> L;
    // (receiver or edge tile, slice) of this workgroup: slice b mod slices on
    // XCD b mod 8, receivers (or edge tiles) in contiguous runs per XCD
    int slice, i, e0, e1;
    if (a.edge_tiles) {
        const int t = xcd_slice_receiver(blockIdx.x, a.num_edge_tiles, a.reverse_slices, slice);
        i = a.edge_tiles[2 * t];
        e0 = a.edge_tiles[2 * t + 1];
        e1 = min(e0 + a.edge_tile, a.graph.first[i + 1]);
    } else {
        i = a.node_offset + xcd_slice_receiver(blockIdx.x, a.node_count, a.reverse_slices, slice);
        e0 = a.graph.first[i];
        e1 = a.graph.first[i + 1];
    }
    const int slices = a.reverse_slices;
    const int k = slice * 64 + static_cast<int>(threadIdx.x);  // < C: C = 64 slices
    const EdgeGraph& g = a.graph;
    const float dcoef = a.d1.table && slice == 0 ? a.d1.dot[i] / a.d1.scale[i] : 0.0f;
    for (int base = e0; base < e1; base += kTile) {
        __syncthreads();
        stage_reverse_tile<S>(a, base, e1, dcoef, L, [&](int e, float d, double rr) {
            double* out = part + 3 * (static_cast<size_t>(e - g.edge_base) * slices + slice);
            const double* x = g.xyz + 3 * static_cast<size_t>(e - g.edge_base);
#pragma unroll
            for (int c = 0; c < 3; ++c) out[c] = static_cast<double>(d * static_cast<float>(x[c] / rr));
        });
        __syncthreads();
        const int count = uniform(L.count);
        (r1_reverse_pass<S, RevGroup<S, G>>(a, i, G == 0, count, k, 0, r1, cg, H1, dPhi1, msg, L), ...);
        __syncthreads();
        if (static_cast<int>(threadIdx.x) < count) {
            const int t = threadIdx.x;
            double p[3] = {0.0, 0.0, 0.0};
            for (int w = 0; w < kForcePartsGrouped; ++w)
                for (int c = 0; c < 3; ++c) p[c] += static_cast<double>(L.f[t][w][c]);
            double f[3];
            tangent_force(p[0], p[1], p[2], L.drop[t], L.geo[t], f);
            double* out = part + 3 * (static_cast<size_t>(L.eid[t] - g.edge_base) * slices + slice);
#pragma unroll
            for (int c = 0; c < 3; ++c) out[c] = -f[c] + static_cast<double>(L.dsc[t] * L.geo[t][c]);
        }
    }
}

// forces[e] = part[e][0] + part[e][1] + ... (slice order), for the edges of
// the launch's receivers (a grid over graph.num_edges, at least their count)
__global__ void __launch_bounds__(256) fold_slices_kernel(LayerArgs a, const double* __restrict__ part,
                                                          double* __restrict__ forces)
{
    const EdgeGraph& g = a.graph;
    const int lo = g.first[a.node_offset] - g.edge_base;
    const int hi = g.first[a.node_offset + a.node_count] - g.edge_base;
    const int e = lo + static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
    if (e >= hi) return;
    const int slices = a.reverse_slices;
    const double* p = part + 3 * static_cast<size_t>(e) * slices;
    double f[3] = {p[0], p[1], p[2]};
    for (int q = 1; q < slices; ++q)
        for (int c = 0; c < 3; ++c) f[c] += p[3 * q + c];
    double* out = forces + 3 * static_cast<size_t>(e);
    for (int c = 0; c < 3; ++c) out[c] = f[c];
}

// ---------------------------------------------------------------------------
// Layer 0 reverse: f_ij += -sum_{lm,k} A0_adj[i,lm,k] (r_hat R0f' Y_lm + R0f dY_lm)
// ---------------------------------------------------------------------------
template <int LMAX, bool kUnfolded>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) a0_reverse_kernel(LayerArgs a, const float* __restrict__ r0f,
                                                          const float* __restrict__ A0,
                                                          const float* __restrict__ A0_adj,
                                                          double* __restrict__ forces)
{
    constexpr int NLM = (LMAX + 1) * (LMAX + 1);
    constexpr int NL = LMAX + 1;
    __shared__ float s_Y[kTile][NLM];
    __shared__ float s_geo[kTile][4];
    __shared__ float s_ir[kTile];  // 1 / r
    __shared__ int s_row[kTile];
    __shared__ int s_h0row[kTile];  // kUnfolded: offset of the source type's H0 row
    __shared__ int s_eid[kTile];
    __shared__ float s_f[kTile][kMaxWaves][3];  // wave sums (stream_ring_sum3)
    __shared__ float s_dsc[kTile];  // A0 density-scale force coefficient per active slot
    __shared__ int s_count;

    int i, t0, t1;  // the receiver and the edges of this workgroup
    block_edges(a, a.edge_tiles_layer0, false, a.edge_tiles_layer0 ? 0 : layer0_receiver(a), i, t0, t1);
    const int k = threadIdx.x;
    const int C = a.C;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int nwaves = blockDim.x >> 6;
    const EdgeGraph& g = a.graph;
    const int voff = min(k, C - 1) * 16;
    const int row_bytes = NL * C * 16;
    float adj[NLM];
    if (k < C) {
        const float* in = A0_adj + static_cast<size_t>(i - a.local_base) * NLM * C + k;
#pragma unroll
        for (int lm = 0; lm < NLM; ++lm) adj[lm] = in[lm * C];
    } else {
#pragma unroll
        for (int lm = 0; lm < NLM; ++lm) adj[lm] = 0.0f;
    }
    const int e0 = g.first[i], e1 = g.first[i + 1];  // all the receiver's edges (density scale)
    // reverse_A0_scaled: dcoef = (A0_adj . A0) / s for the edge terms, adj /= s
    float dcoef = 0.0f;
    if (a.d0.table) {
        __shared__ float s_red[1 + kMaxWaves];
        if (threadIdx.x < 64) {
            const float sc = density_scale(a.d0, g, a.grid, e0, e1);
            if (threadIdx.x == 0) s_red[0] = sc;
        }
        float p = 0.0f;
        if (k < C) {
            const float* f = A0 + static_cast<size_t>(i - a.local_base) * NLM * C + k;
#pragma unroll
            for (int lm = 0; lm < NLM; ++lm) p = fmaf(adj[lm], f[lm * C], p);
        }
        p = wave_sum_dpp(p);
        if (lane == 0) s_red[1 + wave] = p;
        __syncthreads();
        const float sc = s_red[0];
        float dot = 0.0f;
        for (int w = 0; w < nwaves; ++w) dot += s_red[1 + w];
        dcoef = dot / sc;
#pragma unroll
        for (int lm = 0; lm < NLM; ++lm) adj[lm] /= sc;
    }
    // the adjoint contracted with the harmonic gradients, once per receiver:
    // sum_m adj[l, m] dP_lm/dr_k = sum_m' B[k][l - 1][m'] P_{l-1, m'}
    float B[3][LMAX][2 * LMAX - 1];
#pragma unroll
    for (int d = 0; d < 3; ++d)
#pragma unroll
        for (int l = 1; l <= LMAX; ++l)
#pragma unroll
            for (int mp = 0; mp < 2 * l - 1; ++mp) {
                float v = 0.0f;
#pragma unroll
                for (int m = 0; m < 2 * l + 1; ++m)
                    if (kShGrad[d][l * l + m][mp] != 0.0f) v = fmaf(kShGrad[d][l * l + m][mp], adj[l * l + m], v);
                B[d][l - 1][mp] = v;
            }
    for (int base = t0; base < t1; base += kTile) {
        __syncthreads();
        if (threadIdx.x < 64) {
            const int t = threadIdx.x;
            double rr;
            const int n = min(kTile, t1 - base);
            const TileSlot ts = compact_edge<true, false>(g, a.grid, base, n, t, rr, &s_count, kUnfolded);
            const int e = base + t;
            if (ts.active) {
                const int sl = ts.slot;
                edge_harmonics<LMAX, false>(g.xyz + 3 * static_cast<size_t>(e - g.edge_base), rr, s_Y[sl], nullptr,
                                            nullptr, nullptr, s_geo[sl]);
                s_geo[sl][3] = ts.x;
                s_ir[sl] = static_cast<float>(1.0 / rr);
                s_row[sl] = ts.row;
                if constexpr (kUnfolded) s_h0row[sl] = (g.edge_pair[e - g.edge_base] & 0xffff) % g.num_active * C;
                s_eid[sl] = e;
                s_dsc[sl] = a.d0.table ? dcoef * density_slope(a.d0.table, a.grid, g.edge_pair[e - g.edge_base] >> 16, rr) : 0.0f;
            } else if (t < n && a.d0.table) {
                // beyond r_cut: only the density-scale term (reverse_A0_scaled visits every neighbour)
                const float d = dcoef * density_slope(a.d0.table, a.grid, g.edge_pair[e - g.edge_base] >> 16, rr);
                const double* x = g.xyz + 3 * static_cast<size_t>(e - g.edge_base);
                double* out = forces + 3 * static_cast<size_t>(e - g.edge_base);
                out[0] += static_cast<double>(d * static_cast<float>(x[0] / rr));
                out[1] += static_cast<double>(d * static_cast<float>(x[1] / rr));
                out[2] += static_cast<double>(d * static_cast<float>(x[2] / rr));
            }
        }
        __syncthreads();
        const int count = uniform(s_count);
        auto fetch = [&](int j, float4v* c) {
            const auto rs = buffer_rsrc(r0f + static_cast<size_t>(uniform(s_row[j])) * NL * C * 4, row_bytes);
#pragma unroll
            for (int l = 0; l < NL; ++l) c[l] = load4(rs, voff, l * C * 16);
        };
        // with P_lm(r) = r^l Y_lm, d/dr [R_l Y_lm] = r_hat (R_l' - l R_l / r) Y_lm
        // + (R_l / r) sum_m' c_lm,m' Y_{l-1, m'}: the edge force is
        // r_hat A + g with A = sum_l (R_l' - l R_l / r) sum_m adj Y and
        // g_k = sum_l (R_l / r) sum_m' B[k][l - 1][m'] Y_{l-1, m'}
        auto edge_force = [&](int j, const float4v* cl, float& fx, float& fy, float& fz) {
            const float x = uniform(s_geo[j][3]);
            const float ir = uniform(s_ir[j]);
            float Y[NLM], yl[NL];
#pragma unroll
            for (int lm = 0; lm < NLM; ++lm) Y[lm] = s_Y[j][lm];
#pragma unroll
            for (int l = 0; l < NL; ++l) yl[l] = 0.0f;
#pragma unroll
            for (int lm = 0; lm < NLM; ++lm) yl[kLmL[lm]] = fmaf(Y[lm], adj[lm], yl[kLmL[lm]]);
            float A = 0.0f, gx = 0.0f, gy = 0.0f, gz = 0.0f;
#pragma unroll
            for (int l = 0; l < NL; ++l) {
                float R, dR;
                cubic_value_slope(cl[l], x, R, dR);
                if (l == 0) {
                    A = fmaf(dR, yl[0], A);
                } else {
                    A = fmaf(fmaf(-static_cast<float>(l) * ir, R, dR), yl[l], A);
                    float ix = 0.0f, iy = 0.0f, iz = 0.0f;
#pragma unroll
                    for (int mp = 0; mp < 2 * l - 1; ++mp) {
                        const float y = Y[(l - 1) * (l - 1) + mp];
                        ix = fmaf(y, B[0][l - 1][mp], ix);
                        iy = fmaf(y, B[1][l - 1][mp], iy);
                        iz = fmaf(y, B[2][l - 1][mp], iz);
                    }
                    const float h = R * ir;
                    gx = fmaf(h, ix, gx);
                    gy = fmaf(h, iy, gy);
                    gz = fmaf(h, iz, gz);
                }
            }
            fx = fmaf(s_geo[j][0], A, gx);
            fy = fmaf(s_geo[j][1], A, gy);
            fz = fmaf(s_geo[j][2], A, gz);
            if constexpr (kUnfolded) {
                // the edge's terms are linear in its radial values: scale once
                const float h = a.h0[uniform(s_h0row[j]) + min(k, C - 1)];
                fx *= h;
                fy *= h;
                fz *= h;
            }
        };
        auto store = [&](int j, const float (&sums)[3]) {
            s_f[j][wave][0] = sums[0];
            s_f[j][wave][1] = sums[1];
            s_f[j][wave][2] = sums[2];
        };
        float4v ring[kDepth][NL];
        stream_ring_sum3(count, ring, fetch, edge_force, store);
        __syncthreads();
        if (threadIdx.x < count) {
            const int t = threadIdx.x;
            double f[3] = {0.0, 0.0, 0.0};
            for (int w = 0; w < nwaves; ++w)
                for (int c = 0; c < 3; ++c) f[c] += static_cast<double>(s_f[t][w][c]);
            double* out = forces + 3 * static_cast<size_t>(s_eid[t] - g.edge_base);
#pragma unroll
            for (int c = 0; c < 3; ++c) out[c] += -f[c] + static_cast<double>(s_dsc[t] * s_geo[t][c]);
        }
    }
}

// H1 adjoint gather.  A message row (num_LM x C floats) is read as float4s,
// the block's threads covering the whole row.  The source's edge list is
// taken 64 edges at a time: wave 0 reads the edge ids and lengths and
// compacts the edges within r_cut (the others carry no message) into LDS in
// ascending edge order, then every thread streams the listed rows with
// kGatherDepth float4 loads in flight (kGatherDepth / V rows of V float4s)
// -- no load in the streaming loop waits on another.  Rows are summed in
// ascending edge order.  The messages are written with streaming stores and
// read here with non-temporal loads: each is read once, and the 0.8 GB of a
// 5,000-atom call would only churn the L2s (against the default policy:
// gather 188 -> 132 us, the writing R1 reverse 568-577 -> 554-556 us).
constexpr int kGatherStage = 64;
constexpr int kGatherDepth = 16;

// The message (and r) of edge e is row e - g.edge_base.
template <int V>
__device__ __forceinline__ void gather_range(const EdgeGraph& g, double r_cut, const float4* __restrict__ m4,
                                             int row4, int t0, int t1, float4 (&acc)[V])
{
    __shared__ int s_rows[kGatherStage];
    __shared__ int s_n;
    const int tid = threadIdx.x, T = blockDim.x;
    for (int base = t0; base < t1; base += kGatherStage) {
        __syncthreads();  // the previous rows are consumed
        if (tid < 64) {
            const int tt = base + tid;
            bool on = false;
            int row = 0;
            if (tt < t1) {
                row = static_cast<int>(g.tedge[tt] - g.edge_base);
                on = g.r[row] < r_cut;
            }
            const unsigned long long mask = __ballot(on);
            const int slot = __builtin_amdgcn_mbcnt_hi(static_cast<unsigned>(mask >> 32),
                                                       __builtin_amdgcn_mbcnt_lo(static_cast<unsigned>(mask), 0));
            if (on) s_rows[slot] = row;
            if (tid == 0) s_n = __popcll(mask);
        }
        __syncthreads();
        const int n = s_n;
        constexpr int D = kGatherDepth / V > 4 ? kGatherDepth / V : 4;  // rows per thread in flight
        for (int j = 0; j < n; j += D) {
            float4 v[D][V];
#pragma unroll
            for (int u = 0; u < D; ++u)
#pragma unroll
                for (int q = 0; q < V; ++q) {
                    const int c = tid + q * T;
                    v[u][q] = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (j + u < n && c < row4) {
                        const float4v t = __builtin_nontemporal_load(
                            reinterpret_cast<const float4v*>(m4 + static_cast<size_t>(s_rows[j + u]) * row4 + c));
                        v[u][q] = make_float4(t.x, t.y, t.z, t.w);
                    }
                }
#pragma unroll
            for (int u = 0; u < D; ++u)
#pragma unroll
                for (int q = 0; q < V; ++q) {
                    acc[q].x += v[u][q].x;
                    acc[q].y += v[u][q].y;
                    acc[q].z += v[u][q].z;
                    acc[q].w += v[u][q].w;
                }
        }
    }
}

// H1_adj[s] = sum over the edges e with source s (ascending e) of msg[e]
template <int V>
__global__ void __launch_bounds__(256) gather_messages_kernel(LayerArgs a, int row4, const float* __restrict__ msg,
                                                              float* __restrict__ H1_adj)
{
    const int s = a.node_offset + xcd_contiguous(blockIdx.x, a.node_count);
    float4 acc[V];
#pragma unroll
    for (int q = 0; q < V; ++q) acc[q] = make_float4(0.f, 0.f, 0.f, 0.f);
    gather_range<V>(a.graph, a.grid.r_cut, reinterpret_cast<const float4*>(msg), row4, a.graph.tfirst[s],
                    a.graph.tfirst[s + 1], acc);
    float4* out = reinterpret_cast<float4*>(H1_adj) + static_cast<size_t>(s) * row4;
#pragma unroll
    for (int q = 0; q < V; ++q) {
        const int c = threadIdx.x + q * blockDim.x;
        if (c < row4) out[c] = acc[q];
    }
}

// Tiled execution: H1_adj[s] += sum over the run's edges (ascending) of
// msg[e - edge_base]; one workgroup per run of the tile, runs of one tile have
// distinct sources.
template <int V>
__global__ void __launch_bounds__(256) gather_tile_runs_kernel(LayerArgs a, TileRuns runs, int row4,
                                                               const float* __restrict__ msg,
                                                               float* __restrict__ H1_adj)
{
    const int run = blockIdx.x;
    const int t0 = runs.start[run];
    float4 acc[V];
#pragma unroll
    for (int q = 0; q < V; ++q) acc[q] = make_float4(0.f, 0.f, 0.f, 0.f);
    gather_range<V>(a.graph, a.grid.r_cut, reinterpret_cast<const float4*>(msg), row4, t0, t0 + runs.length[run],
                    acc);
    float4* out = reinterpret_cast<float4*>(H1_adj) + static_cast<size_t>(runs.source[run]) * row4;
#pragma unroll
    for (int q = 0; q < V; ++q) {
        const int c = threadIdx.x + q * blockDim.x;
        if (c < row4) {
            float4 o = out[c];
            o.x += acc[q].x;
            o.y += acc[q].y;
            o.z += acc[q].z;
            o.w += acc[q].w;
            out[c] = o;
        }
    }
}

__global__ void add_direct_kernel(int nodes, int C, int nLM, const float* __restrict__ direct,
                                  float* __restrict__ M0_adj)
{
    const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= static_cast<size_t>(nodes) * C) return;
    const size_t i = idx / C, k = idx % C;
    M0_adj[i * nLM * C + k] += direct[idx];
}

// ---------------------------------------------------------------------------
// geometry and reductions
// ---------------------------------------------------------------------------
// Cartesian vector of the fractional vector f in the cell (rows = lattice
// vectors), with explicit fused operations so that every kernel forms it
// with the same rounding.
__device__ __forceinline__ void fractional_to_cartesian(const double f[3], const double* __restrict__ cell,
                                                        double out[3])
{
    for (int c = 0; c < 3; ++c) out[c] = fma(f[2], cell[6 + c], fma(f[1], cell[3 + c], f[0] * cell[c]));
}

// Reference vector of edge e (receiver i, source j) of a prepared geometry.
// A device-built graph (g.built) keeps its fractional positions and cell
// shifts; its fractional edge vector is formed as the build formed it --
// the positions wrapped to [0, 1) (p - floor(p)), their difference, plus the
// image shift + floor(p_j) - floor(p_i) -- so it equals the build's stored
// vector bit for bit.
__device__ __forceinline__ void reference_edge(const GeometryRef& g, const double* __restrict__ cell, size_t e,
                                               size_t i, size_t j, double ref[3])
{
    if (g.edges) {
        const double* f = g.edges + 3 * e;
        if (g.fractional) {
            const double fv[3] = {f[0], f[1], f[2]};
            fractional_to_cartesian(fv, cell, ref);
        } else {
            ref[0] = f[0], ref[1] = f[1], ref[2] = f[2];
        }
        return;
    }
    int sh[3];
    for (int a = 0; a < 3; ++a) sh[a] = g.shifts8 ? static_cast<int>(g.shifts8[3 * e + a]) : g.shifts[3 * e + a];
    const double* pj = g.positions + 3 * j;
    const double* pi = g.positions + 3 * i;
    if (g.built) {
        double d[3];
        for (int a = 0; a < 3; ++a) {
            const double fj = floor(pj[a]), fi = floor(pi[a]);
            const int image = sh[a] + static_cast<int>(fj) - static_cast<int>(fi);
            d[a] = ((pj[a] - fj) - (pi[a] - fi)) + static_cast<double>(image);
        }
        fractional_to_cartesian(d, cell, ref);
    } else if (g.fractional) {
        double d[3];
        for (int a = 0; a < 3; ++a) d[a] = pj[a] - pi[a] + static_cast<double>(sh[a]);
        fractional_to_cartesian(d, cell, ref);
    } else {
        // single_layer_tiled_edge_geometry, mace_kokkos_factorized_lifecycle.cpp:1858-1866
        for (int c = 0; c < 3; ++c) {
            ref[c] = pj[c] - pi[c];
            for (int a = 0; a < 3; ++a) ref[c] += static_cast<double>(sh[a]) * cell[3 * a + c];
        }
    }
}

__global__ void edge_geometry_kernel(int E, const int* __restrict__ receiver,
                                     const int* __restrict__ source, GeometryRef g,
                                     const double* __restrict__ disp, const double* __restrict__ cell,
                                     double r_cut, double* __restrict__ xyz, double* __restrict__ r,
                                     unsigned long long* __restrict__ invalid)
{
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const size_t i = receiver[e], j = source[e];
    double ref[3];
    reference_edge(g, cell, static_cast<size_t>(e), i, j, ref);
    double v[3];
    for (int c = 0; c < 3; ++c) v[c] = ref[c] + disp[3 * j + c] - disp[3 * i + c];
    const double d2 = v[0] * v[0] + v[1] * v[1] + v[2] * v[2];
    if (!(d2 > 0.0) || !(d2 < 1.0e300)) {
        atomicAdd(invalid, 1ull);
        v[0] = r_cut;
        v[1] = 0.0;
        v[2] = 0.0;
    }
    xyz[3 * static_cast<size_t>(e)] = v[0];
    xyz[3 * static_cast<size_t>(e) + 1] = v[1];
    xyz[3 * static_cast<size_t>(e) + 2] = v[2];
    r[e] = sqrt(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
}

// F_a = sum_{e: src=a} f_e - sum_{e: recv=a} f_e.  One wave per atom; lane l
// sums edges l, l+64, ... of each list, then a fixed butterfly combines the
// lanes, so the result does not depend on scheduling.
__global__ void __launch_bounds__(256) atom_forces_kernel(int N, const int* __restrict__ first,
                                                          const int* __restrict__ tfirst,
                                                          const int* __restrict__ tedge,
                                                          const double* __restrict__ f,
                                                          double* __restrict__ out)
{
    const int lane = threadIdx.x & 63;
    const int a = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (a >= N) return;
    double acc[3] = {0.0, 0.0, 0.0};
    for (int t = tfirst[a] + lane; t < tfirst[a + 1]; t += 64) {
        const size_t e = tedge[t];
        acc[0] += f[3 * e], acc[1] += f[3 * e + 1], acc[2] += f[3 * e + 2];
    }
    for (int e = first[a] + lane; e < first[a + 1]; e += 64) {
        acc[0] -= f[3 * static_cast<size_t>(e)], acc[1] -= f[3 * static_cast<size_t>(e) + 1],
            acc[2] -= f[3 * static_cast<size_t>(e) + 2];
    }
    for (int off = 32; off > 0; off >>= 1)
        for (int c = 0; c < 3; ++c) acc[c] += __shfl_xor(acc[c], off, 64);
    if (lane == 0) {
        out[3 * static_cast<size_t>(a)] = acc[0];
        out[3 * static_cast<size_t>(a) + 1] = acc[1];
        out[3 * static_cast<size_t>(a) + 2] = acc[2];
    }
}

constexpr int kReduceThreads = 256;
constexpr int kReduceItems = 4;  // items per thread per block

// partials[b][0] = sum of energies of block b's nodes, [1..9] = -(1/V) f (x) xyz
__global__ void __launch_bounds__(kReduceThreads) totals_partial_kernel(
    int N, int E, const double* __restrict__ energies, const double* __restrict__ f,
    const double* __restrict__ xyz, double inv_volume, double* __restrict__ partials)
{
    __shared__ double s[kReduceThreads][10];
    const int t = threadIdx.x;
    double acc[10];
    for (int c = 0; c < 10; ++c) acc[c] = 0.0;
    const size_t span = static_cast<size_t>(kReduceThreads) * kReduceItems;
    const size_t b0 = static_cast<size_t>(blockIdx.x) * span;
    for (int q = 0; q < kReduceItems; ++q) {
        const size_t idx = b0 + static_cast<size_t>(q) * kReduceThreads + t;
        if (idx < static_cast<size_t>(N)) acc[0] += energies[idx];
        if (idx < static_cast<size_t>(E)) {
            for (int c = 0; c < 9; ++c)
                acc[1 + c] += -inv_volume * f[3 * idx + c / 3] * xyz[3 * idx + c % 3];
        }
    }
    for (int c = 0; c < 10; ++c) s[t][c] = acc[c];
    __syncthreads();
    for (int w = kReduceThreads / 2; w > 0; w >>= 1) {
        if (t < w)
            for (int c = 0; c < 10; ++c) s[t][c] += s[t + w][c];
        __syncthreads();
    }
    if (t < 10) partials[static_cast<size_t>(blockIdx.x) * 10 + t] = s[0][t];
}

__global__ void __launch_bounds__(256) totals_final_kernel(int num_partials,
                                                         const double* __restrict__ partials,
                                                         double* __restrict__ out, int accumulate)
{
    __shared__ double s[256][10];
    const int t = threadIdx.x;
    double acc[10];
    for (int c = 0; c < 10; ++c) acc[c] = 0.0;
    for (int b = t; b < num_partials; b += 256)
        for (int c = 0; c < 10; ++c) acc[c] += partials[static_cast<size_t>(b) * 10 + c];
    for (int c = 0; c < 10; ++c) s[t][c] = acc[c];
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (t < w)
            for (int c = 0; c < 10; ++c) s[t][c] += s[t + w][c];
        __syncthreads();
    }
    if (t < 10) out[t] = accumulate ? out[t] + s[0][t] : s[0][t];
}

// ZBL pair term of every neighbour (zbl_kokkos.cpp:76-126, 154-201): one wave
// per receiver, lanes over its edges; the energy partial sums are combined
// by a fixed butterfly, so the result does not depend on scheduling.
__global__ void __launch_bounds__(256) zbl_kernel(int node_begin, int N, const int* __restrict__ first,
                                                  long long edge_base, const int* __restrict__ edge_pair,
                                                  const double* __restrict__ xyz, const double* __restrict__ r,
                                                  ZblArgs z, double* __restrict__ energies,
                                                  double* __restrict__ forces)
{
    const int lane = threadIdx.x & 63;
    const int local = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (local >= N) return;
    const int i = node_begin + local;
    const int p = z.p;
    const double k0 = (p + 1.0) * (p + 2.0) / 2.0, k1 = p * (p + 2.0), k2 = p * (p + 1.0) / 2.0;
    double energy = 0.0;
    for (int ge = first[i] + lane; ge < first[i + 1]; ge += 64) {
        const long long e = ge - edge_base;  // index into the per-edge arrays
        const int po = edge_pair[e] & 0xffff;
        const double rr = r[e];
        const double r_max = z.r_max[po];
        if (rr >= r_max) continue;
        const double inverse_a = z.inverse_a[po];
        const double r_over_a = rr * inverse_a;
        const double e0 = z.c[0] * exp(-3.2 * r_over_a);
        const double e1 = z.c[1] * exp(-0.9423 * r_over_a);
        const double e2 = z.c[2] * exp(-0.4028 * r_over_a);
        const double e3 = z.c[3] * exp(-0.2016 * r_over_a);
        const double phi = e0 + e1 + e2 + e3;
        const double dphi = inverse_a * (-3.2 * e0 - 0.9423 * e1 - 0.4028 * e2 - 0.2016 * e3);
        const double inverse_r = 1.0 / rr;
        const double bare = z.prefactor[po] * inverse_r * phi;
        const double bare_gradient = z.prefactor[po] * inverse_r * inverse_r * (rr * dphi - phi);
        const double x = rr / r_max;
        double xpm1 = 1.0;
        for (int q = 0; q < p - 1; ++q) xpm1 *= x;
        const double xp = xpm1 * x, xp1 = xp * x, xp2 = xp1 * x;
        const double envelope = 1.0 - k0 * xp + k1 * xp1 - k2 * xp2;
        const double envelope_gradient = (-k0 * p * xpm1 + k1 * (p + 1.0) * xp - k2 * (p + 2.0) * xp1) / r_max;
        energy += 0.5 * bare * envelope;
        const double gradient = 0.5 * (bare * envelope_gradient + bare_gradient * envelope);
        double* f = forces + 3 * static_cast<size_t>(e);
        const double* v = xyz + 3 * static_cast<size_t>(e);
        f[0] -= v[0] / rr * gradient;
        f[1] -= v[1] / rr * gradient;
        f[2] -= v[2] / rr * gradient;
    }
    for (int off = 32; off > 0; off >>= 1) energy += __shfl_xor(energy, off, 64);
    if (lane == 0) energies[i] += energy;
}

// Tiled execution: the geometry of one tile's edges in the reused arena --
// edge vector, length and pair code of edge e at index e - edge_base.  One
// wave per receiver, lanes over its edges.  The vector is the reference
// vector of the prepared geometry plus the displacement difference, as
// edge_geometry_kernel forms it graph-wide; with in_arena the caller's
// vectors are already in place and only the pair codes are formed.
__global__ void __launch_bounds__(256) tile_geometry_kernel(TileGeometry g)
{
    const int lane = threadIdx.x & 63;
    const int local = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (local >= g.node_count) return;
    const int i = g.node_begin + local;
    const int a = g.type_active[g.node_types[i]];
    for (int e = g.first[i] + lane; e < g.first[i + 1]; e += 64) {
        const size_t le = static_cast<size_t>(e - g.edge_base);
        const size_t j = g.source[e];
        if (!g.in_arena) {
            double ref[3];
            reference_edge(g.ref, g.cell, static_cast<size_t>(e), static_cast<size_t>(i), j, ref);
            double v[3];
            for (int c = 0; c < 3; ++c) v[c] = ref[c] + g.disp[3 * j + c] - g.disp[3 * static_cast<size_t>(i) + c];
            const double d2 = v[0] * v[0] + v[1] * v[1] + v[2] * v[2];
            if (!(d2 > 0.0) || !(d2 < 1.0e300)) {
                if (g.invalid) atomicAdd(g.invalid, 1ull);
                v[0] = g.r_cut;
                v[1] = 0.0;
                v[2] = 0.0;
            }
            g.xyz[3 * le] = v[0];
            g.xyz[3 * le + 1] = v[1];
            g.xyz[3 * le + 2] = v[2];
            g.r[le] = sqrt(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
        }
        if (g.pair_source) {
            g.edge_pair[le] = g.pair_source[e];
        } else {
            const int b = g.type_active[g.node_types[j]];
            const int po = a * g.num_active + b;
            const int pu = g.shared_tables ? 0 : unordered_pair(a, b, g.num_active);
            g.edge_pair[le] = po | (pu << 16);
        }
    }
}

// Tiled execution: a tile's directed forces into the atom forces, in a fixed
// order.  Receiver part: F[i] -= sum over the receiver's edges (one wave per
// receiver, lanes over edges, fixed butterfly).  Source part: F[s] += sum
// over each source run of the tile (one wave per run; the runs of a tile have
// distinct sources, and both launches run in stream order).
__global__ void __launch_bounds__(256) fold_receiver_forces_kernel(int node_begin, int N, const int* __restrict__ first,
                                                                   long long edge_base, const double* __restrict__ f,
                                                                   double* __restrict__ out)
{
    const int lane = threadIdx.x & 63;
    const int local = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (local >= N) return;
    const int i = node_begin + local;
    double acc[3] = {0.0, 0.0, 0.0};
    for (int e = first[i] + lane; e < first[i + 1]; e += 64) {
        const size_t le = static_cast<size_t>(e - edge_base);
        acc[0] += f[3 * le], acc[1] += f[3 * le + 1], acc[2] += f[3 * le + 2];
    }
    for (int off = 32; off > 0; off >>= 1)
        for (int c = 0; c < 3; ++c) acc[c] += __shfl_xor(acc[c], off, 64);
    if (lane == 0)
        for (int c = 0; c < 3; ++c) out[3 * static_cast<size_t>(i) + c] -= acc[c];
}

__global__ void __launch_bounds__(256) fold_source_runs_kernel(TileRuns runs, const int* __restrict__ tedge,
                                                               long long edge_base, const double* __restrict__ f,
                                                               double* __restrict__ out)
{
    const int lane = threadIdx.x & 63;
    const int run = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (run >= runs.count) return;
    const int t0 = runs.start[run], t1 = t0 + runs.length[run];
    double acc[3] = {0.0, 0.0, 0.0};
    for (int t = t0 + lane; t < t1; t += 64) {
        const size_t le = static_cast<size_t>(tedge[t] - edge_base);
        acc[0] += f[3 * le], acc[1] += f[3 * le + 1], acc[2] += f[3 * le + 2];
    }
    for (int off = 32; off > 0; off >>= 1)
        for (int c = 0; c < 3; ++c) acc[c] += __shfl_xor(acc[c], off, 64);
    if (lane == 0)
        for (int c = 0; c < 3; ++c) out[3 * static_cast<size_t>(runs.source[run]) + c] += acc[c];
}

__global__ void fill_f64_kernel(double* __restrict__ out, long long n, double value)
{
    for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<long long>(gridDim.x) * blockDim.x)
        out[i] = value;
}

inline int node_threads(int C) { return ((C + 63) / 64) * 64; }

}  // namespace

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
hipError_t launch_a0_forward(const LayerArgs& a, const float* r0f, float* A0, hipStream_t s)
{
    if (a.node_count <= 0) return hipSuccess;
    const int threads = node_threads(a.C);
    const bool u = a.h0 != nullptr;
    if (a.a0_slices > 1) {
        if ((a.a0_slices != 2 && a.a0_slices != 4) || a.C != 64 * a.a0_slices) return hipErrorInvalidValue;
        const int blocks = a.node_count * a.a0_slices;
        switch (a.l_max) {
        case 2:
            if (u) a0_forward_sliced_kernel<2, true><<<blocks, 256, 0, s>>>(a, r0f, A0), note_launch();
            else a0_forward_sliced_kernel<2, false><<<blocks, 256, 0, s>>>(a, r0f, A0), note_launch();
            break;
        case 3:
            if (u) a0_forward_sliced_kernel<3, true><<<blocks, 256, 0, s>>>(a, r0f, A0), note_launch();
            else a0_forward_sliced_kernel<3, false><<<blocks, 256, 0, s>>>(a, r0f, A0), note_launch();
            break;
        default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    switch (a.l_max) {
    case 2:
        if (u) a0_forward_kernel<2, true><<<a.node_count, threads, 0, s>>>(a, r0f, A0), note_launch();
        else a0_forward_kernel<2, false><<<a.node_count, threads, 0, s>>>(a, r0f, A0), note_launch();
        break;
    case 3:
        if (u) a0_forward_kernel<3, true><<<a.node_count, threads, 0, s>>>(a, r0f, A0), note_launch();
        else a0_forward_kernel<3, false><<<a.node_count, threads, 0, s>>>(a, r0f, A0), note_launch();
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Workgroups of an edge kernel: one per edge tile with a tile list (the
// whole graph only), else one per receiver.
static int edge_blocks(const LayerArgs& a, const int* tiles, bool& ok)
{
    ok = !tiles || (a.node_offset == 0 && a.local_base == 0 && a.node_count == a.graph.num_nodes &&
                    a.edge_tile > 0 && a.edge_tile <= kTile);
    return tiles ? a.num_edge_tiles : a.node_count;
}

hipError_t launch_a0_reverse(const LayerArgs& a, const float* r0f, const float* A0, const float* A0_adj,
                             double* forces, hipStream_t s)
{
    if (a.node_count <= 0) return hipSuccess;
    const int threads = node_threads(a.C);
    const bool u = a.h0 != nullptr;
    bool ok;
    const int blocks = edge_blocks(a, a.edge_tiles_layer0, ok);
    if (!ok) return hipErrorInvalidValue;
    if (blocks <= 0) return hipSuccess;
    switch (a.l_max) {
    case 2:
        if (u) a0_reverse_kernel<2, true><<<blocks, threads, 0, s>>>(a, r0f, A0, A0_adj, forces), note_launch();
        else a0_reverse_kernel<2, false><<<blocks, threads, 0, s>>>(a, r0f, A0, A0_adj, forces), note_launch();
        break;
    case 3:
        if (u) a0_reverse_kernel<3, true><<<blocks, threads, 0, s>>>(a, r0f, A0, A0_adj, forces), note_launch();
        else a0_reverse_kernel<3, false><<<blocks, threads, 0, s>>>(a, r0f, A0, A0_adj, forces), note_launch();
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_r1_forward(const LayerArgs& a, const float* r1, const float* cg, const float* H1,
                             float* Phi1, hipStream_t s)
{
    if (a.node_count <= 0) return hipSuccess;
    const int slices = a.channel_slices;
    if (slices != 1 && (a.C != 64 * slices || (slices != 2 && slices != 4))) return hipErrorInvalidValue;
    const int threads = node_threads(a.C);
    const int blocks = a.node_count * slices;
    if (a.l_max == 2 && a.L_max == 1)
        r1_forward_kernel<R1Shape<2, 1>><<<a.node_count, threads, 0, s>>>(a, r1, cg, H1, Phi1), note_launch();
    else if (a.l_max == 3 && a.L_max == 1 && slices == 1)
        r1_forward_kernel<R1Shape<3, 1>><<<a.node_count, threads, 0, s>>>(a, r1, cg, H1, Phi1), note_launch();
    else if (a.l_max == 3 && a.L_max == 1)
        r1_forward_sliced_kernel<R1Shape<3, 1>><<<blocks, 256, 0, s>>>(a, r1, cg, H1, Phi1), note_launch();
    else if (a.l_max == 3 && a.L_max == 2 && slices == 1)
        r1_forward_kernel<R1Shape<3, 2>><<<a.node_count, threads, 0, s>>>(a, r1, cg, H1, Phi1), note_launch();
    else if (a.l_max == 3 && a.L_max == 2)
        r1_forward_sliced_kernel<R1Shape<3, 2>><<<blocks, 256, 0, s>>>(a, r1, cg, H1, Phi1), note_launch();
    else if (a.l_max == 3 && a.L_max == 0)
        r1_forward_kernel<R1Shape<3, 0>><<<a.node_count, threads, 0, s>>>(a, r1, cg, H1, Phi1), note_launch();
    else if (a.l_max == 2 && a.L_max == 0)
        r1_forward_kernel<R1Shape<2, 0>><<<a.node_count, threads, 0, s>>>(a, r1, cg, H1, Phi1), note_launch();
    else if (a.l_max == 2 && a.L_max == 2)
        r1_forward_kernel<R1Shape<2, 2>><<<a.node_count, threads, 0, s>>>(a, r1, cg, H1, Phi1), note_launch();
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

// the (3, 2) reverse runs passes 0 and 1: the generated source-l2 groups
static_assert(R1Groups<3, 2>::NREV == 2, "reverse pass list out of date");

hipError_t launch_r1_reverse(const LayerArgs& a, const float* r1, const float* cg, const float* H1,
                             const float* dPhi1, double* forces, float* msg, double* part, hipStream_t s)
{
    if (a.node_count <= 0) return hipSuccess;
    const int threads = node_threads(a.C);
    if (threads > 256) return hipErrorInvalidValue;
    if (a.reverse_slices > 1) {
        if (!part || !r1_reverse_sliceable(a.l_max, a.L_max, a.C, a.reverse_slices)) return hipErrorInvalidValue;
        // one-wave workgroups per (receiver or edge tile, slice)
        bool ok;
        const int units = edge_blocks(a, a.edge_tiles, ok);
        if (!ok) return hipErrorInvalidValue;
        if (units > 0)
            r1_reverse_sliced_kernel<R1Shape<3, 2>, 0, 1><<<units * a.reverse_slices, 64, 0, s>>>(
                a, r1, cg, H1, dPhi1, part, msg), note_launch();
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
        if (a.graph.num_edges > 0)
            fold_slices_kernel<<<(a.graph.num_edges + 255) / 256, 256, 0, s>>>(a, part, forces), note_launch();
        return hipGetLastError();
    }
    // the single-pass kernels take edge tiles; the (3, 2) path-group kernel
    // runs one workgroup per receiver
    bool ok;
    const int blocks = edge_blocks(a, a.edge_tiles, ok);
    if (!ok) return hipErrorInvalidValue;
    if (a.l_max == 3 && a.L_max == 2) {
        LayerArgs ar = a;
        ar.edge_tiles = nullptr;
        r1_reverse_grouped_kernel<R1Shape<3, 2>, 0, 1><<<a.node_count, threads, 0, s>>>(ar, r1, cg, H1, dPhi1,
                                                                                       forces, msg), note_launch();
        return hipGetLastError();
    }
    if (blocks <= 0) return hipSuccess;
    if (a.l_max == 2 && a.L_max == 1)
        r1_reverse_kernel<R1Shape<2, 1>><<<blocks, threads, 0, s>>>(a, r1, cg, H1, dPhi1, forces, msg),
            note_launch();
    else if (a.l_max == 3 && a.L_max == 1)
        r1_reverse_kernel<R1Shape<3, 1>><<<blocks, threads, 0, s>>>(a, r1, cg, H1, dPhi1, forces, msg),
            note_launch();
    else if (a.l_max == 3 && a.L_max == 0)
        r1_reverse_kernel<R1Shape<3, 0>><<<blocks, threads, 0, s>>>(a, r1, cg, H1, dPhi1, forces, msg),
            note_launch();
    else if (a.l_max == 2 && a.L_max == 0)
        r1_reverse_kernel<R1Shape<2, 0>><<<blocks, threads, 0, s>>>(a, r1, cg, H1, dPhi1, forces, msg),
            note_launch();
    else if (a.l_max == 2 && a.L_max == 2)
        r1_reverse_kernel<R1Shape<2, 2>><<<blocks, threads, 0, s>>>(a, r1, cg, H1, dPhi1, forces, msg),
            note_launch();
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

// threads and float4s per thread covering one message row of num_LM x C floats
static void gather_shape(const LayerArgs& a, int& row4, int& threads, int& per_thread)
{
    const int nLM = (a.L_max + 1) * (a.L_max + 1);
    row4 = nLM * a.C / 4;
    threads = std::min(256, ((row4 + 63) / 64) * 64);
    per_thread = (row4 + threads - 1) / threads;
}

hipError_t launch_gather_messages(const LayerArgs& a, const float* msg, float* H1_adj, hipStream_t s)
{
    if (a.node_count <= 0) return hipSuccess;
    if (a.C % 4 != 0) return hipErrorInvalidValue;
    int row4, threads, v;
    gather_shape(a, row4, threads, v);
    switch (v) {
    case 1: gather_messages_kernel<1><<<a.node_count, threads, 0, s>>>(a, row4, msg, H1_adj), note_launch(); break;
    case 2: gather_messages_kernel<2><<<a.node_count, threads, 0, s>>>(a, row4, msg, H1_adj), note_launch(); break;
    case 3: gather_messages_kernel<3><<<a.node_count, threads, 0, s>>>(a, row4, msg, H1_adj), note_launch(); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gather_tile_runs(const LayerArgs& a, const TileRuns& runs, const float* msg,
                                   float* H1_adj, hipStream_t s)
{
    if (runs.count <= 0) return hipSuccess;
    if (a.C % 4 != 0) return hipErrorInvalidValue;
    int row4, threads, v;
    gather_shape(a, row4, threads, v);
    switch (v) {
    case 1: gather_tile_runs_kernel<1><<<runs.count, threads, 0, s>>>(a, runs, row4, msg, H1_adj), note_launch(); break;
    case 2: gather_tile_runs_kernel<2><<<runs.count, threads, 0, s>>>(a, runs, row4, msg, H1_adj), note_launch(); break;
    case 3: gather_tile_runs_kernel<3><<<runs.count, threads, 0, s>>>(a, runs, row4, msg, H1_adj), note_launch(); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_add_direct(int nodes, int C, int num_LM, const float* direct, float* M0_adj,
                             hipStream_t s)
{
    const size_t n = static_cast<size_t>(nodes) * C;
    if (n == 0) return hipSuccess;
    add_direct_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, s>>>(nodes, C, num_LM, direct,
                                                                            M0_adj), note_launch();
    return hipGetLastError();
}

hipError_t launch_zbl(int node_begin, int num_nodes, const int* first, long long edge_base, const int* edge_pair,
                      const double* xyz, const double* r, const ZblArgs& z, double* energies, double* forces,
                      hipStream_t s)
{
    if (num_nodes <= 0) return hipSuccess;
    zbl_kernel<<<(num_nodes + 3) / 4, 256, 0, s>>>(node_begin, num_nodes, first, edge_base, edge_pair, xyz, r, z,
                                                   energies, forces), note_launch();
    return hipGetLastError();
}

hipError_t launch_tile_geometry(const TileGeometry& g, hipStream_t s)
{
    if (g.node_count <= 0) return hipSuccess;
    if (!g.in_arena && !g.ref.edges && !((g.ref.shifts || g.ref.shifts8) && g.ref.positions))
        return hipErrorInvalidValue;
    tile_geometry_kernel<<<(g.node_count + 3) / 4, 256, 0, s>>>(g), note_launch();
    return hipGetLastError();
}

hipError_t launch_fold_tile_forces(int node_begin, int node_count, const int* first, const TileRuns& runs,
                                   const int* tedge, long long edge_base, const double* forces, double* atom_forces,
                                   hipStream_t s)
{
    if (node_count > 0)
        fold_receiver_forces_kernel<<<(node_count + 3) / 4, 256, 0, s>>>(node_begin, node_count, first, edge_base,
                                                                         forces, atom_forces), note_launch();
    if (runs.count > 0)
        fold_source_runs_kernel<<<(runs.count + 3) / 4, 256, 0, s>>>(runs, tedge, edge_base, forces, atom_forces), note_launch();
    return hipGetLastError();
}

hipError_t launch_fill_f64(double* out, long long n, double value, hipStream_t s)
{
    if (n <= 0) return hipSuccess;
    const long long blocks = std::min<long long>((n + 255) / 256, 65536);
    fill_f64_kernel<<<static_cast<int>(blocks), 256, 0, s>>>(out, n, value), note_launch();
    return hipGetLastError();
}

hipError_t launch_edge_geometry(int num_edges, const int* receiver, const int* source, const GeometryRef& ref,
                                const double* displacements, const double* cell, double r_cut, double* xyz, double* r,
                                unsigned long long* invalid, hipStream_t s)
{
    if (num_edges <= 0) return hipSuccess;
    if (!ref.edges && !((ref.shifts || ref.shifts8) && ref.positions)) return hipErrorInvalidValue;
    edge_geometry_kernel<<<(num_edges + 255) / 256, 256, 0, s>>>(num_edges, receiver, source, ref, displacements,
                                                                 cell, r_cut, xyz, r, invalid), note_launch();
    return hipGetLastError();
}

hipError_t launch_atom_forces(int num_nodes, const int* first, const int* tfirst, const int* tedge,
                              const double* forces, double* atom_forces, hipStream_t s)
{
    if (num_nodes <= 0) return hipSuccess;
    atom_forces_kernel<<<(num_nodes + 3) / 4, 256, 0, s>>>(num_nodes, first, tfirst, tedge, forces,
                                                           atom_forces), note_launch();
    return hipGetLastError();
}

int reduce_totals_partials(int num_nodes, int num_edges)
{
    const long long n = std::max<long long>(std::max(num_nodes, num_edges), 1);
    const long long span = static_cast<long long>(kReduceThreads) * kReduceItems;
    return static_cast<int>((n + span - 1) / span);
}

hipError_t launch_reduce_totals(int num_nodes, int num_edges, const double* energies,
                                const double* forces, const double* xyz, double inv_volume,
                                double* partials, int num_partials, double* out, hipStream_t s, bool accumulate)
{
    totals_partial_kernel<<<num_partials, kReduceThreads, 0, s>>>(num_nodes, num_edges, energies, forces,
                                                                  xyz, inv_volume, partials), note_launch();
    totals_final_kernel<<<1, 256, 0, s>>>(num_partials, partials, out, accumulate ? 1 : 0), note_launch();
    return hipGetLastError();
}

}  // namespace sxl
