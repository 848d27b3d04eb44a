// gfx950 node kernels: the symmetric contraction M0 (forward and reverse) and
// the readout with its reverse (M1, H2, node energies, the direct scalar
// adjoint and the A1 adjoint).
//
// A workgroup owns one block of nodes of a single element type (nodes grouped
// by type on the host); each thread owns one channel of every node of the
// block.  The polynomial terms of the compiled monomial table are unrolled,
// so a channel's inputs, outputs and gradients stay in registers and each
// coefficient a thread loads is applied to all nodes of the block.  Terms of
// the model JSON without a compiled slot run in a short runtime loop over an
// LDS copy of the inputs, so every monomial table is evaluated exactly.
//
// Reference semantics (libsymmetrix/source/mace.cpp): compute_M0
// :1638-1662, reverse_M0 :1664-1688 (MultivariatePolynomial evaluation and
// gradient, multivariate_polynomial.cpp:10-130), compute_M1 / compute_H2 /
// compute_readouts and reverse_H2 / reverse_M1 :2460-2657 (m0_composite
// basis: H2 = T_z^T M0_scalar + W^T M1, E = E0 + q . M0_scalar + MLP(H2)).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <utility>

#include "device_math.hpp"
#include "kernels.hpp"
#include "poly_shapes.inc"

namespace sxl {
namespace {

inline int node_threads(int C) { return ((C + 63) / 64) * 64; }

// ---------------------------------------------------------------------------
// compiled terms (registers)
//
// The term code is expanded at compile time (one instantiation per term), in
// chunks of kChunk terms: the coefficients of chunk i + 1 are loaded while
// chunk i is evaluated.  Between chunks a scheduling barrier keeps the
// compiler from hoisting every load to the top, and the inputs pass through
// an empty asm statement so that products of inputs are shared only within a
// chunk (shared across the whole polynomial they would exhaust the register
// file).
// ---------------------------------------------------------------------------
constexpr int kChunk = 16;

template <int NB, int NIN>
__device__ __forceinline__ void chunk_boundary(float (&x)[NB][NIN])
{
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int n = 0; n < NB; ++n)
#pragma unroll
        for (int v = 0; v < NIN; ++v) asm volatile("" : "+v"(x[n][v]));
}

// kQuad: the compiled coefficients lie in runs of four terms per channel
// ([slot / 4][C][4]), one 16-byte load per lane bringing four terms; else one
// [slot][C] row per term.  voff is the lane's byte offset in a [slot][C] row
// (kk * 4).  The M0 kernels take the runs of four (medium shape: forward
// 32.6 -> 24 us, reverse 51 -> 43 us); the readout keeps a row per term, as
// its eight-node blocks (graphs of many receivers) then need 256 VGPRs and
// run at one wave per SIMD (0.81 -> 1.30 ms on water) or spill at two
// (0.81 -> 0.82 ms), and its two-node blocks gain nothing.
template <class P, int BASE, bool kQuad>
__device__ __forceinline__ void load_chunk(__amdgpu_buffer_rsrc_t cs, int voff, int C, float (&c)[kChunk])
{
    static_assert(BASE % 4 == 0 && kChunk % 4 == 0);
    if constexpr (!kQuad) {
#pragma unroll
        for (int j = 0; j < kChunk; ++j) c[j] = BASE + j < P::NT ? load1(cs, voff, (BASE + j) * C * 4) : 0.0f;
        return;
    }
#pragma unroll
    for (int u = 0; u < kChunk / 4; ++u) {
        if (BASE + 4 * u < P::NT) {
            const float4v q = load4(cs, 4 * voff, (BASE / 4 + u) * C * 16);
            c[4 * u] = q.x;
            c[4 * u + 1] = q.y;
            c[4 * u + 2] = q.z;
            c[4 * u + 3] = q.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) c[4 * u + j] = 0.0f;
        }
    }
}

// The compiled tables list consecutive groups of terms of one output and
// degree that share a lead: all of a monomial's indices but its free index
// lz (la for degree 2, la and lb for degree 3).  A group is evaluated
// nested: U = sum_t c_t x[lz_t], then out += lead * U with lead = x[la] or
// x[la] x[lb] -- one FMA per term instead of a product and an FMA.  The
// gradient of a group is dx[lz_t] += (lam lead) c_t per term and, once per
// group, dx[la] += lam U (degree 2) or dx[la] += lam U x[lb] and
// dx[lb] += lam U x[la] (degree 3).
template <class P>
struct PolyGroups {
    static constexpr bool same(int s, int t)
    {
        return P::out[s] == P::out[t] && P::deg[s] == P::deg[t] && P::deg[t] >= 2 && P::la[s] == P::la[t] &&
               (P::deg[t] == 2 || P::lb[s] == P::lb[t]);
    }
    static constexpr bool first(int t) { return t == 0 || !same(t - 1, t); }
    static constexpr bool last(int t) { return t == P::NT - 1 || !same(t, t + 1); }
};

template <class P, int NB, int T>
__device__ __forceinline__ void term_value(float c, const float (&x)[NB][P::NIN], float (&out)[NB][P::NOUT],
                                           float (&U)[NB])
{
    if constexpr (T < P::NT) {
        constexpr int d = P::deg[T], a0 = P::la[T], a1 = P::lb[T], z = P::lz[T], o = P::out[T];
        constexpr bool f = PolyGroups<P>::first(T), l = PolyGroups<P>::last(T);
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            if constexpr (d == 1) {
                out[n][o] = fmaf(c, x[n][a0], out[n][o]);
            } else {
                U[n] = f ? c * x[n][z] : fmaf(c, x[n][z], U[n]);
                if constexpr (l) {
                    const float lead = d == 2 ? x[n][a0] : x[n][a0] * x[n][a1];
                    out[n][o] = fmaf(lead, U[n], out[n][o]);
                }
            }
        }
    }
}

template <class P, int NB, int T>
__device__ __forceinline__ void term_gradient(float c, const float (&x)[NB][P::NIN], const float (&lam)[NB][P::NOUT],
                                              float (&g)[NB][P::NIN], float (&U)[NB], float (&pl)[NB])
{
    if constexpr (T < P::NT) {
        constexpr int d = P::deg[T], a0 = P::la[T], a1 = P::lb[T], z = P::lz[T], o = P::out[T];
        constexpr bool f = PolyGroups<P>::first(T), l = PolyGroups<P>::last(T);
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            if constexpr (d == 1) {
                g[n][a0] = fmaf(c, lam[n][o], g[n][a0]);
            } else {
                if constexpr (f) pl[n] = d == 2 ? lam[n][o] * x[n][a0] : lam[n][o] * (x[n][a0] * x[n][a1]);
                U[n] = f ? c * x[n][z] : fmaf(c, x[n][z], U[n]);
                g[n][z] = fmaf(pl[n], c, g[n][z]);
                if constexpr (l) {
                    const float q = lam[n][o] * U[n];
                    if constexpr (d == 2) {
                        g[n][a0] += q;
                    } else {
                        g[n][a0] = fmaf(q, x[n][a1], g[n][a0]);
                        g[n][a1] = fmaf(q, x[n][a0], g[n][a1]);
                    }
                }
            }
        }
    }
}

template <class P, int NB, int BASE, int... J>
__device__ __forceinline__ void value_chunk(const float (&c)[kChunk], const float (&x)[NB][P::NIN],
                                            float (&out)[NB][P::NOUT], float (&U)[NB], std::integer_sequence<int, J...>)
{
    (term_value<P, NB, BASE + J>(c[J], x, out, U), ...);
}

template <class P, int NB, int BASE, int... J>
__device__ __forceinline__ void gradient_chunk(const float (&c)[kChunk], const float (&x)[NB][P::NIN],
                                               const float (&lam)[NB][P::NOUT], float (&g)[NB][P::NIN],
                                               float (&U)[NB], float (&pl)[NB], std::integer_sequence<int, J...>)
{
    (term_gradient<P, NB, BASE + J>(c[J], x, lam, g, U, pl), ...);
}

template <class P, int NB, int BASE, bool kQuad>
__device__ __forceinline__ void core_value_from(__amdgpu_buffer_rsrc_t cs, int voff, int C, const float (&cur)[kChunk],
                                                float (&x)[NB][P::NIN], float (&out)[NB][P::NOUT], float (&U)[NB])
{
    if constexpr (BASE < P::NT) {
        float nxt[kChunk];
        if constexpr (BASE + kChunk < P::NT) load_chunk<P, BASE + kChunk, kQuad>(cs, voff, C, nxt);
        value_chunk<P, NB, BASE>(cur, x, out, U, std::make_integer_sequence<int, kChunk>{});
        chunk_boundary<NB, P::NIN>(x);
        core_value_from<P, NB, BASE + kChunk, kQuad>(cs, voff, C, nxt, x, out, U);
    }
}

template <class P, int NB, int BASE, bool kQuad>
__device__ __forceinline__ void core_gradient_from(__amdgpu_buffer_rsrc_t cs, int voff, int C,
                                                   const float (&cur)[kChunk], float (&x)[NB][P::NIN],
                                                   const float (&lam)[NB][P::NOUT], float (&g)[NB][P::NIN],
                                                   float (&U)[NB], float (&pl)[NB])
{
    if constexpr (BASE < P::NT) {
        float nxt[kChunk];
        if constexpr (BASE + kChunk < P::NT) load_chunk<P, BASE + kChunk, kQuad>(cs, voff, C, nxt);
        gradient_chunk<P, NB, BASE>(cur, x, lam, g, U, pl, std::make_integer_sequence<int, kChunk>{});
        chunk_boundary<NB, P::NIN>(x);
        core_gradient_from<P, NB, BASE + kChunk, kQuad>(cs, voff, C, nxt, x, lam, g, U, pl);
    }
}

// out[n][o] += sum over compiled terms t of output o: c_t prod x[n][i]
template <class P, int NB, bool kQuad>
__device__ __forceinline__ void core_value(__amdgpu_buffer_rsrc_t cs, int voff, int C,
                                           float (&x)[NB][P::NIN], float (&out)[NB][P::NOUT])
{
    if constexpr (P::NT > 0) {
        float c[kChunk], U[NB];
        load_chunk<P, 0, kQuad>(cs, voff, C, c);
        core_value_from<P, NB, 0, kQuad>(cs, voff, C, c, x, out, U);
    }
}

// g[n][i] += sum over compiled terms t: c_t lam[n][out_t] d(prod x[n])/dx_i
template <class P, int NB, bool kQuad>
__device__ __forceinline__ void core_gradient(__amdgpu_buffer_rsrc_t cs, int voff, int C,
                                              float (&x)[NB][P::NIN], const float (&lam)[NB][P::NOUT],
                                              float (&g)[NB][P::NIN])
{
    if constexpr (P::NT > 0) {
        float c[kChunk], U[NB], pl[NB];
        load_chunk<P, 0, kQuad>(cs, voff, C, c);
        core_gradient_from<P, NB, 0, kQuad>(cs, voff, C, c, x, lam, g, U, pl);
    }
}

// ---------------------------------------------------------------------------
// remainder terms (runtime table; one node, inputs in this thread's LDS column)
// ---------------------------------------------------------------------------
template <int NOUT>
__device__ __forceinline__ void rem_value(const PolyArgs& p, __amdgpu_buffer_rsrc_t cs, int voff, int C,
                                          int first_rem, const float* xc, int xs, float (&f)[NOUT])
{
#pragma unroll
    for (int o = 0; o < NOUT; ++o)
        for (int t = p.rem_offsets[o]; t < p.rem_offsets[o + 1]; ++t) {
            const int pk = p.rem_packed[t];
            const int d = pk & 15;
            float v = xc[((pk >> 4) & 63) * xs];
            if (d > 1) v *= xc[((pk >> 10) & 63) * xs];
            if (d > 2) v *= xc[((pk >> 16) & 63) * xs];
            f[o] = fmaf(load1(cs, voff, (first_rem + t) * C * 4), v, f[o]);
        }
}

template <int NOUT>
__device__ __forceinline__ void rem_gradient(const PolyArgs& p, __amdgpu_buffer_rsrc_t cs, int voff, int C,
                                             int first_rem, const float* xc, float* gc, int xs,
                                             const float (&lam)[NOUT])
{
#pragma unroll
    for (int o = 0; o < NOUT; ++o)
        for (int t = p.rem_offsets[o]; t < p.rem_offsets[o + 1]; ++t) {
            const int pk = p.rem_packed[t];
            const int d = pk & 15;
            const int a0 = ((pk >> 4) & 63) * xs, a1 = ((pk >> 10) & 63) * xs, a2 = ((pk >> 16) & 63) * xs;
            const float u = load1(cs, voff, (first_rem + t) * C * 4) * lam[o];
            if (d == 1) {
                gc[a0] += u;
            } else if (d == 2) {
                const float x0 = xc[a0], x1 = xc[a1];
                gc[a0] += u * x1;
                gc[a1] += u * x0;
            } else {
                const float x0 = xc[a0], x1 = xc[a1], x2 = xc[a2];
                gc[a0] += u * (x1 * x2);
                gc[a1] += u * (x0 * x2);
                gc[a2] += u * (x0 * x1);
            }
        }
}

// First remainder slot of a coefficient block.
template <class P, bool kQuad>
constexpr int first_rem_slot() { return kQuad ? compiled_slots(P::NT) : P::NT; }

// Forward remainder of the NB nodes held in registers (LDS column of NIN floats).
template <class P, int NB, bool kQuad>
__device__ __forceinline__ void rem_value_nodes(const PolyArgs& p, __amdgpu_buffer_rsrc_t cs, int voff, int C,
                                                float* xc, int xs, const float (&x)[NB][P::NIN],
                                                float (&out)[NB][P::NOUT])
{
#pragma unroll
    for (int n = 0; n < NB; ++n) {
#pragma unroll
        for (int v = 0; v < P::NIN; ++v) xc[v * xs] = x[n][v];
        rem_value<P::NOUT>(p, cs, voff, C, first_rem_slot<P, kQuad>(), xc, xs, out[n]);
    }
}

template <class P, int NB, bool kQuad>
__device__ __forceinline__ void rem_gradient_nodes(const PolyArgs& p, __amdgpu_buffer_rsrc_t cs, int voff, int C,
                                                   float* xc, float* gc, int xs, const float (&x)[NB][P::NIN],
                                                   const float (&lam)[NB][P::NOUT], float (&g)[NB][P::NIN])
{
#pragma unroll
    for (int n = 0; n < NB; ++n) {
#pragma unroll
        for (int v = 0; v < P::NIN; ++v) {
            xc[v * xs] = x[n][v];
            gc[v * xs] = 0.0f;
        }
        rem_gradient<P::NOUT>(p, cs, voff, C, first_rem_slot<P, kQuad>(), xc, gc, xs, lam[n]);
#pragma unroll
        for (int v = 0; v < P::NIN; ++v) g[n][v] += gc[v * xs];
    }
}

// ---------------------------------------------------------------------------
// M0 forward / reverse
// ---------------------------------------------------------------------------
template <class P, int NB>
__global__ void __launch_bounds__(256) m0_forward_kernel(LayerArgs a, PolyArgs p, NodeBlocks nb,
                                                          const float* __restrict__ A0, float* __restrict__ M0)
{
    constexpr int NIN = P::NIN, NOUT = P::NOUT;
    extern __shared__ float s_mem[];  // remainder terms only: [NIN][blockDim.x]
    const NodeBlock blk = nb.blocks[nb.first + blockIdx.x];
    const int k = threadIdx.x;
    const int C = a.C;
    const int kk = min(k, C - 1);
    int node[NB];
    float x[NB][NIN];
#pragma unroll
    for (int n = 0; n < NB; ++n) {
        node[n] = n < blk.count ? nb.order[blk.start + n] - a.local_base : -1;
        const float* in = A0 + static_cast<size_t>(max(node[n], 0)) * NIN * C + kk;
#pragma unroll
        for (int v = 0; v < NIN; ++v) x[n][v] = node[n] >= 0 ? in[v * C] : 0.0f;
    }
    float out[NB][NOUT];
#pragma unroll
    for (int n = 0; n < NB; ++n)
#pragma unroll
        for (int o = 0; o < NOUT; ++o) out[n][o] = 0.0f;
    const auto cs = buffer_rsrc(p.coef + static_cast<size_t>(blk.type) * p.stride * C, p.stride * C * 4);
    core_value<P, NB, true>(cs, kk * 4, C, x, out);
    if (p.num_rem > 0) rem_value_nodes<P, NB, true>(p, cs, kk * 4, C, s_mem + k, blockDim.x, x, out);
    if (k < C) {
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            if (node[n] < 0) continue;
            float* o = M0 + static_cast<size_t>(node[n]) * NOUT * C + k;
#pragma unroll
            for (int q = 0; q < NOUT; ++q) o[q * C] = out[n][q];
        }
    }
}

template <class P, int NB>
__global__ void __launch_bounds__(256) m0_reverse_kernel(LayerArgs a, PolyArgs p, NodeBlocks nb,
                                                          const float* __restrict__ A0,
                                                          const float* __restrict__ M0_adj,
                                                          float* __restrict__ A0_adj)
{
    constexpr int NIN = P::NIN, NOUT = P::NOUT;
    extern __shared__ float s_mem[];  // remainder terms only: [2][NIN][blockDim.x]
    const NodeBlock blk = nb.blocks[nb.first + blockIdx.x];
    const int k = threadIdx.x;
    const int C = a.C;
    const int kk = min(k, C - 1);
    int node[NB];
    float x[NB][NIN], lam[NB][NOUT], g[NB][NIN];
#pragma unroll
    for (int n = 0; n < NB; ++n) {
        node[n] = n < blk.count ? nb.order[blk.start + n] - a.local_base : -1;
        const size_t row = static_cast<size_t>(max(node[n], 0));
        const float* in = A0 + row * NIN * C + kk;
        const float* la = M0_adj + row * NOUT * C + kk;
#pragma unroll
        for (int v = 0; v < NIN; ++v) {
            x[n][v] = node[n] >= 0 ? in[v * C] : 0.0f;
            g[n][v] = 0.0f;
        }
#pragma unroll
        for (int o = 0; o < NOUT; ++o) lam[n][o] = node[n] >= 0 ? la[o * C] : 0.0f;
    }
    const auto cs = buffer_rsrc(p.coef + static_cast<size_t>(blk.type) * p.stride * C, p.stride * C * 4);
    core_gradient<P, NB, true>(cs, kk * 4, C, x, lam, g);
    if (p.num_rem > 0)
        rem_gradient_nodes<P, NB, true>(p, cs, kk * 4, C, s_mem + k, s_mem + NIN * blockDim.x + k, blockDim.x, x,
                                  lam, g);
    if (k < C) {
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            if (node[n] < 0) continue;
            float* o = A0_adj + static_cast<size_t>(node[n]) * NIN * C + k;
#pragma unroll
            for (int v = 0; v < NIN; ++v) o[v * C] = g[n][v];
        }
    }
}

// ---------------------------------------------------------------------------
// Readout and its reverse, NB nodes of one type per workgroup:
//   1. M1[n][k] = P1(A1[n][:, k]), xs[n][k] = M0[n][0][k]          (LDS)
//   2. H2[n][k] = sum_in T[in][k] xs[n][in] + W[in][k] M1[n][in]  (LDS)
//   3. hidden units, one thread per (node, unit): z = W1[h] . H2[n],
//      act = W2[h] s silu(z), dact = W2[h] s silu'(z)
//   4. E[n] = E0 + q . xs[n] + sum_h act; H2_adj[n][k] = sum_h dact W1[h][k]
//   5. direct[n][k] = q[k] + sum_o T[k][o] H2_adj[n][o];
//      M1_adj[n][k] = sum_o W[k][o] H2_adj[n][o]
//   6. A1_adj[n][lm][k] = M1_adj[n][k] dP1/dA1[lm]
// ---------------------------------------------------------------------------
// Weight streaming of the readout's matrix-vector phases.  A phase reads its
// weights (column k of the thread, or one row) in blocks of W floats; the
// blocks pass through a ring of kStreamRing register buffers so
// the loads of the next kStreamRing - 1 blocks are in flight while one block
// is consumed (waiting on each block's loads in turn would put one memory
// round trip per block on the critical path).  `load(b, buf)` fills buf with
// block b (clamped to the last block: every step issues the same loads, so
// the waits stay exact), `use(b, buf)` consumes it.  Blocks beyond the last
// whole ring round are handled by `tail(b)` without the ring.
constexpr int kStreamRing = 4;

template <int W, class Load, class Use, class Tail>
__device__ __forceinline__ void stream_blocks(int nblocks, Load& load, Use& use, Tail& tail)
{
    constexpr int R = kStreamRing;
    float ring[R][W];
    const int full = nblocks / R * R;
    if (full > 0) {
#pragma unroll
        for (int d = 0; d < R - 1; ++d) load(d, ring[d]);
        for (int b0 = 0; b0 < full; b0 += R) {
#pragma unroll
            for (int d = 0; d < R; ++d) {
                load(min(b0 + d + R - 1, full - 1), ring[(d + R - 1) % R]);
                use(b0 + d, ring[d]);
            }
        }
    }
    for (int b = full; b < nblocks; ++b) tail(b);
}

constexpr int kReadoutGroup = 4;  // nodes held in registers by the polynomial phases
constexpr int kMaxHidden = 64;
constexpr int kMaxWavesReadout = 4;  // 256 threads

template <class P1, int NB>
__global__ void __launch_bounds__(256) readout_kernel(ReadoutArgs a)
{
    constexpr int NIN = P1::NIN;
    constexpr int G = NB < kReadoutGroup ? NB : kReadoutGroup;
    static_assert(NB % G == 0, "readout block must hold whole register groups");
    extern __shared__ float s_mem[];
    const int T = blockDim.x;  // >= C, a multiple of 64
    float* s_xs = s_mem;                // [NB][T]
    float* s_m1 = s_xs + NB * T;        // [NB][T]
    float* s_h2 = s_m1 + NB * T;        // [NB][T]: H2, then its adjoint
    float* s_act = s_h2 + NB * T;       // [NB][kMaxHidden]
    float* s_gh = s_act + NB * kMaxHidden;  // [NB][kMaxHidden]
    float* s_rem = s_gh + NB * kMaxHidden;  // [2][NIN][T], remainder terms only
    const NodeBlock blk = a.nodes.blocks[a.nodes.first + blockIdx.x];
    const int k = threadIdx.x;
    const int C = a.C;
    const int kk = min(k, C - 1);
    const bool ok = k < C;
    const int H = a.hidden;
    int node[NB];
#pragma unroll
    for (int n = 0; n < NB; ++n) node[n] = n < blk.count ? a.nodes.order[blk.start + n] : -1;
    const auto cs = buffer_rsrc(a.p1.coef + static_cast<size_t>(blk.type) * a.p1.stride * C,
                                a.p1.stride * C * 4);
    const int voff = kk * 4;

    // A1 density scale of each node (compute_A1_scaled, mace.cpp:2381-2402)
    float dscale[NB];
#pragma unroll
    for (int n = 0; n < NB; ++n) dscale[n] = (a.a1_scale && node[n] >= 0) ? a.a1_scale[node[n]] : 1.0f;

    // 1. M1 and the scalar M0 block
#pragma unroll
    for (int g0 = 0; g0 < NB; g0 += G) {
        float x[G][NIN], m1[G][1];
#pragma unroll
        for (int n = 0; n < G; ++n) {
            const int i = node[g0 + n];
            const float* in = a.A1 + static_cast<size_t>(max(i - a.local_base, 0)) * NIN * C + kk;
#pragma unroll
            for (int v = 0; v < NIN; ++v) x[n][v] = i >= 0 ? in[v * C] : 0.0f;
            if (a.a1_scale) {
#pragma unroll
                for (int v = 0; v < NIN; ++v) x[n][v] /= dscale[g0 + n];
            }
            m1[n][0] = 0.0f;
        }
        core_value<P1, G, false>(cs, voff, C, x, m1);
        if (a.p1.num_rem > 0) rem_value_nodes<P1, G, false>(a.p1, cs, voff, C, s_rem + k, T, x, m1);
#pragma unroll
        for (int n = 0; n < G; ++n) {
            const int i = node[g0 + n];
            const bool on = ok && i >= 0;
            s_m1[(g0 + n) * T + k] = on ? m1[n][0] : 0.0f;
            s_xs[(g0 + n) * T + k] = on ? a.M0[static_cast<size_t>(i) * a.m0_stride + k] : 0.0f;
        }
    }
    __syncthreads();

    // 2. H2 (weight columns streamed, 4 inputs per block); per-wave partial
    //    sums of q . xs for the energies
    if (ok) {
        float h2[NB];
#pragma unroll
        for (int n = 0; n < NB; ++n) h2[n] = 0.0f;
        // weights in runs of four inputs per output ([in / 4][out][4]): two
        // 16-byte loads per lane and block of four inputs
        const float4* Tm = reinterpret_cast<const float4*>(a.H2M0 + static_cast<size_t>(blk.type) * C * C) + k;
        const float4* Wm = reinterpret_cast<const float4*>(a.H2M1) + k;
        auto load = [&](int b, float (&w)[8]) {
            const float4 t = Tm[static_cast<size_t>(b) * C], m = Wm[static_cast<size_t>(b) * C];
            w[0] = t.x, w[1] = t.y, w[2] = t.z, w[3] = t.w;
            w[4] = m.x, w[5] = m.y, w[6] = m.z, w[7] = m.w;
        };
        auto use = [&](int b, const float (&w)[8]) {
            const int in = 4 * b;
#pragma unroll
            for (int n = 0; n < NB; ++n) {
                const float4 xv = *reinterpret_cast<const float4*>(s_xs + n * T + in);
                const float4 mv = *reinterpret_cast<const float4*>(s_m1 + n * T + in);
                float h = h2[n];
                h = fmaf(w[0], xv.x, h);
                h = fmaf(w[1], xv.y, h);
                h = fmaf(w[2], xv.z, h);
                h = fmaf(w[3], xv.w, h);
                h = fmaf(w[4], mv.x, h);
                h = fmaf(w[5], mv.y, h);
                h = fmaf(w[6], mv.z, h);
                h = fmaf(w[7], mv.w, h);
                h2[n] = h;
            }
        };
        auto tail = [&](int b) {
            float w[8];
            load(b, w);
            use(b, w);
        };
        stream_blocks<8>(C / 4, load, use, tail);
#pragma unroll
        for (int n = 0; n < NB; ++n) s_h2[n * T + k] = h2[n];
    }
    __shared__ float s_e1[kMaxWavesReadout][NB];
    {
        const float qk = ok ? a.q[k] : 0.0f;
        const int wv = threadIdx.x >> 6;
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            const float e = partial_sum_dpp<1>(ok ? qk * s_xs[n * T + k] : 0.0f);
            if ((threadIdx.x & 63) == 63) s_e1[wv][n] = e;
        }
    }
    __syncthreads();

    // 3. hidden layer of readout_2
    for (int job = threadIdx.x; job < NB * H; job += T) {
        const int n = job / H, h = job - (job / H) * H;
        const float* w1 = a.W1 + static_cast<size_t>(h) * C;
        const float* hn = s_h2 + n * T;
        float z = 0.0f;
        // the weight row streamed in blocks of 4 (C is a multiple of 4)
        auto load = [&](int b, float (&w)[4]) {
            const float4 v = *reinterpret_cast<const float4*>(w1 + 4 * b);
            w[0] = v.x;
            w[1] = v.y;
            w[2] = v.z;
            w[3] = v.w;
        };
        auto use = [&](int b, const float (&w)[4]) {
            const float4 hv = *reinterpret_cast<const float4*>(hn + 4 * b);
            z = fmaf(w[0], hv.x, z);
            z = fmaf(w[1], hv.y, z);
            z = fmaf(w[2], hv.z, z);
            z = fmaf(w[3], hv.w, z);
        };
        auto tail = [&](int b) {
            float w[4];
            load(b, w);
            use(b, w);
        };
        stream_blocks<4>(C / 4, load, use, tail);
        const float sig = 1.0f / (1.0f + expf(-z));
        const float act = a.scale * z * sig;
        const float dact = a.scale * sig + a.scale * z * sig * (1.0f - sig);
        s_act[n * kMaxHidden + h] = a.W2[h] * act;
        s_gh[n * kMaxHidden + h] = a.W2[h] * dact;
    }
    __syncthreads();

    // 4. energies (one thread per node) and the H2 adjoint
    if (threadIdx.x < blk.count) {
        const int n = threadIdx.x;
        const int i = a.nodes.order[blk.start + n];
        float e1 = 0.0f;
        for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) e1 += s_e1[w][n];
        float e2 = 0.0f;
        for (int h = 0; h < H; ++h) e2 += s_act[n * kMaxHidden + h];
        a.energies[i] = a.E0[blk.type] + static_cast<double>(e1) + static_cast<double>(e2);
    }
    if (ok) {
        float gh2[NB];
#pragma unroll
        for (int n = 0; n < NB; ++n) gh2[n] = 0.0f;
        for (int h = 0; h < H; ++h) {
            const float w = a.W1[static_cast<size_t>(h) * C + k];
#pragma unroll
            for (int n = 0; n < NB; ++n) gh2[n] = fmaf(s_gh[n * kMaxHidden + h], w, gh2[n]);
        }
        // H2 is dead (its last reader, step 3, finished at the barrier above)
#pragma unroll
        for (int n = 0; n < NB; ++n) s_h2[n * T + k] = gh2[n];
    }
    __syncthreads();

    // 5. direct scalar adjoint and the M1 adjoint
    float m1adj[NB];
#pragma unroll
    for (int n = 0; n < NB; ++n) m1adj[n] = 0.0f;
    if (ok) {
        float d[NB];
        const float qk = a.q[k];
#pragma unroll
        for (int n = 0; n < NB; ++n) d[n] = qk;
        const float4* Tt = reinterpret_cast<const float4*>(a.H2M0T + static_cast<size_t>(blk.type) * C * C) + k;
        const float4* Wt = reinterpret_cast<const float4*>(a.H2M1T) + k;
        auto load = [&](int b, float (&w)[8]) {
            const float4 t = Tt[static_cast<size_t>(b) * C], m = Wt[static_cast<size_t>(b) * C];
            w[0] = t.x, w[1] = t.y, w[2] = t.z, w[3] = t.w;
            w[4] = m.x, w[5] = m.y, w[6] = m.z, w[7] = m.w;
        };
        auto use = [&](int b, const float (&w)[8]) {
            const int o = 4 * b;
#pragma unroll
            for (int n = 0; n < NB; ++n) {
                const float4 gv = *reinterpret_cast<const float4*>(s_h2 + n * T + o);
                d[n] = fmaf(w[0], gv.x, d[n]);
                d[n] = fmaf(w[1], gv.y, d[n]);
                d[n] = fmaf(w[2], gv.z, d[n]);
                d[n] = fmaf(w[3], gv.w, d[n]);
                m1adj[n] = fmaf(w[4], gv.x, m1adj[n]);
                m1adj[n] = fmaf(w[5], gv.y, m1adj[n]);
                m1adj[n] = fmaf(w[6], gv.z, m1adj[n]);
                m1adj[n] = fmaf(w[7], gv.w, m1adj[n]);
            }
        };
        auto tail = [&](int b) {
            float w[8];
            load(b, w);
            use(b, w);
        };
        stream_blocks<8>(C / 4, load, use, tail);
#pragma unroll
        for (int n = 0; n < NB; ++n)
            if (node[n] >= 0) a.direct[static_cast<size_t>(node[n]) * C + k] = d[n];
    }

    // 6. A1 adjoint; for a scaled model also A1_adj . A1 per node and the
    //    adjoint of the unscaled A1 (reverse_A1_scaled, mace.cpp:2404-2458)
    __shared__ float s_dot[kMaxWavesReadout][NB];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int g0 = 0; g0 < NB; g0 += G) {
        float x[G][NIN], lam[G][1], g[G][NIN];
#pragma unroll
        for (int n = 0; n < G; ++n) {
            const int i = node[g0 + n];
            const float* in = a.A1 + static_cast<size_t>(max(i - a.local_base, 0)) * NIN * C + kk;
#pragma unroll
            for (int v = 0; v < NIN; ++v) {
                x[n][v] = i >= 0 ? in[v * C] : 0.0f;
                g[n][v] = 0.0f;
            }
            if (a.a1_scale) {
#pragma unroll
                for (int v = 0; v < NIN; ++v) x[n][v] /= dscale[g0 + n];
            }
            lam[n][0] = m1adj[g0 + n];
        }
        core_gradient<P1, G, false>(cs, voff, C, x, lam, g);
        if (a.p1.num_rem > 0)
            rem_gradient_nodes<P1, G, false>(a.p1, cs, voff, C, s_rem + k, s_rem + NIN * T + k, T, x, lam, g);
        if (a.a1_scale) {
#pragma unroll
            for (int n = 0; n < G; ++n) {
                float p = 0.0f;
                if (ok) {
#pragma unroll
                    for (int v = 0; v < NIN; ++v) p = fmaf(g[n][v], x[n][v], p);
                }
                p = wave_sum_dpp(p);
                if (lane == 0) s_dot[wave][g0 + n] = p;
            }
        }
        if (ok) {
#pragma unroll
            for (int n = 0; n < G; ++n) {
                const int i = node[g0 + n];
                if (i < 0) continue;
                float* out = a.A1_adj + static_cast<size_t>(i - a.local_base) * NIN * C + k;
#pragma unroll
                for (int v = 0; v < NIN; ++v) out[v * C] = a.a1_scale ? g[n][v] / dscale[g0 + n] : g[n][v];
            }
        }
    }
    if (a.a1_scale) {
        __syncthreads();
        if (threadIdx.x < blk.count) {
            const int n = threadIdx.x;
            float dot = 0.0f;
            for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) dot += s_dot[w][n];
            a.a1_dot[a.nodes.order[blk.start + n]] = dot;
        }
    }
}

template <int LIN, int LOUT, int CORR>
hipError_t m0_forward_launch(const LayerArgs& a, const PolyArgs& p, const NodeBlocks& nb, const float* A0,
                             float* M0, hipStream_t s)
{
    using P = PolyShape<LIN, LOUT, CORR>;
    if (nb.block_nodes < 1 || nb.block_nodes > kM0ForwardBlockNodesWide) return hipErrorInvalidValue;
    const int threads = node_threads(a.C);
    const size_t shmem = p.num_rem > 0 ? sizeof(float) * P::NIN * threads : 0;
    // the kernel holds at least as many nodes as the list's largest block
    if (nb.block_nodes == 1)
        m0_forward_kernel<P, 1><<<nb.count, threads, shmem, s>>>(a, p, nb, A0, M0), note_launch();
    else if (nb.block_nodes <= kM0BlockNodes)
        m0_forward_kernel<P, kM0BlockNodes><<<nb.count, threads, shmem, s>>>(a, p, nb, A0, M0), note_launch();
    else
        m0_forward_kernel<P, kM0ForwardBlockNodesWide><<<nb.count, threads, shmem, s>>>(a, p, nb, A0, M0),
            note_launch();
    return hipGetLastError();
}

template <int LIN, int LOUT, int CORR>
hipError_t m0_reverse_launch(const LayerArgs& a, const PolyArgs& p, const NodeBlocks& nb, const float* A0,
                             const float* M0_adj, float* A0_adj, hipStream_t s)
{
    using P = PolyShape<LIN, LOUT, CORR>;
    const int threads = node_threads(a.C);
    const size_t shmem = p.num_rem > 0 ? sizeof(float) * 2 * P::NIN * threads : 0;
    // the kernel holds at least as many nodes as the list's largest block
    if (nb.block_nodes == 1)
        m0_reverse_kernel<P, 1><<<nb.count, threads, shmem, s>>>(a, p, nb, A0, M0_adj, A0_adj), note_launch();
    else if (nb.block_nodes > 1 && nb.block_nodes <= kM0ReverseBlockNodesNarrow)
        m0_reverse_kernel<P, kM0ReverseBlockNodesNarrow><<<nb.count, threads, shmem, s>>>(a, p, nb, A0, M0_adj,
                                                                                          A0_adj), note_launch();
    else if (nb.block_nodes > kM0ReverseBlockNodesNarrow && nb.block_nodes <= kM0BlockNodes)
        m0_reverse_kernel<P, kM0BlockNodes><<<nb.count, threads, shmem, s>>>(a, p, nb, A0, M0_adj, A0_adj),
            note_launch();
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

template <int LIN, int CORR>
hipError_t readout_launch(const ReadoutArgs& a, hipStream_t s)
{
    using P = PolyShape<LIN, 0, CORR>;
    const int threads = std::max(node_threads(a.C), 64);
    // the kernel holds at least as many nodes as the list's largest block;
    // its LDS is laid out for the kernel's capacity
    const int most = a.nodes.block_nodes;
    if (most < 1 || most > kReadoutBlockNodes) return hipErrorInvalidValue;
    const size_t NB = most == 1 ? 1 : most <= kReadoutBlockNodesNarrow ? kReadoutBlockNodesNarrow : kReadoutBlockNodes;
    size_t floats = 3 * NB * threads + 2 * NB * kMaxHidden;
    if (a.p1.num_rem > 0) floats += 2 * static_cast<size_t>(P::NIN) * threads;
    if (NB == 1)
        readout_kernel<P, 1><<<a.nodes.count, threads, sizeof(float) * floats, s>>>(a), note_launch();
    else if (NB == kReadoutBlockNodesNarrow)
        readout_kernel<P, kReadoutBlockNodesNarrow><<<a.nodes.count, threads, sizeof(float) * floats, s>>>(a),
            note_launch();
    else
        readout_kernel<P, kReadoutBlockNodes><<<a.nodes.count, threads, sizeof(float) * floats, s>>>(a),
            note_launch();
    return hipGetLastError();
}

}  // namespace

hipError_t launch_m0_forward(const LayerArgs& a, const PolyArgs& p0, const NodeBlocks& nb, const float* A0,
                             float* M0, hipStream_t s)
{
    if (nb.count <= 0) return hipSuccess;
    if (node_threads(a.C) > 256) return hipErrorInvalidValue;
    switch (a.l_max * 100 + a.L_max * 10 + p0.core) {
    case 212: return m0_forward_launch<2, 1, 2>(a, p0, nb, A0, M0, s);
    case 313: return m0_forward_launch<3, 1, 3>(a, p0, nb, A0, M0, s);
    case 323: return m0_forward_launch<3, 2, 3>(a, p0, nb, A0, M0, s);
    case 303: return m0_forward_launch<3, 0, 3>(a, p0, nb, A0, M0, s);
    case 210: return m0_forward_launch<2, 1, 0>(a, p0, nb, A0, M0, s);
    case 310: return m0_forward_launch<3, 1, 0>(a, p0, nb, A0, M0, s);
    case 320: return m0_forward_launch<3, 2, 0>(a, p0, nb, A0, M0, s);
    case 300: return m0_forward_launch<3, 0, 0>(a, p0, nb, A0, M0, s);
    case 202: return m0_forward_launch<2, 0, 2>(a, p0, nb, A0, M0, s);
    case 200: return m0_forward_launch<2, 0, 0>(a, p0, nb, A0, M0, s);
    case 222: return m0_forward_launch<2, 2, 2>(a, p0, nb, A0, M0, s);
    case 220: return m0_forward_launch<2, 2, 0>(a, p0, nb, A0, M0, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_m0_reverse(const LayerArgs& a, const PolyArgs& p0, const NodeBlocks& nb, const float* A0,
                             const float* M0_adj, float* A0_adj, hipStream_t s)
{
    if (nb.count <= 0) return hipSuccess;
    if (node_threads(a.C) > 256) return hipErrorInvalidValue;
    switch (a.l_max * 100 + a.L_max * 10 + p0.core) {
    case 212: return m0_reverse_launch<2, 1, 2>(a, p0, nb, A0, M0_adj, A0_adj, s);
    case 313: return m0_reverse_launch<3, 1, 3>(a, p0, nb, A0, M0_adj, A0_adj, s);
    case 323: return m0_reverse_launch<3, 2, 3>(a, p0, nb, A0, M0_adj, A0_adj, s);
    case 303: return m0_reverse_launch<3, 0, 3>(a, p0, nb, A0, M0_adj, A0_adj, s);
    case 210: return m0_reverse_launch<2, 1, 0>(a, p0, nb, A0, M0_adj, A0_adj, s);
    case 310: return m0_reverse_launch<3, 1, 0>(a, p0, nb, A0, M0_adj, A0_adj, s);
    case 320: return m0_reverse_launch<3, 2, 0>(a, p0, nb, A0, M0_adj, A0_adj, s);
    case 300: return m0_reverse_launch<3, 0, 0>(a, p0, nb, A0, M0_adj, A0_adj, s);
    case 202: return m0_reverse_launch<2, 0, 2>(a, p0, nb, A0, M0_adj, A0_adj, s);
    case 200: return m0_reverse_launch<2, 0, 0>(a, p0, nb, A0, M0_adj, A0_adj, s);
    case 222: return m0_reverse_launch<2, 2, 2>(a, p0, nb, A0, M0_adj, A0_adj, s);
    case 220: return m0_reverse_launch<2, 2, 0>(a, p0, nb, A0, M0_adj, A0_adj, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_readout(const ReadoutArgs& a, hipStream_t s)
{
    if (a.nodes.count <= 0) return hipSuccess;
    if (node_threads(a.C) > 256 || a.hidden > kMaxHidden || a.C % 4 != 0) return hipErrorInvalidValue;
    const int lin = a.num_lm == 9 ? 2 : a.num_lm == 16 ? 3 : -1;
    switch (lin * 10 + a.p1.core) {
    case 22: return readout_launch<2, 2>(a, s);
    case 33: return readout_launch<3, 3>(a, s);
    case 20: return readout_launch<2, 0>(a, s);
    case 30: return readout_launch<3, 0>(a, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace sxl
