// Launch interface between the host evaluator and the gfx950 kernels.
//
// Data layout in HBM (channels fastest everywhere, so a workgroup whose
// threads own channels reads and writes whole 128-byte lines):
//   node features   A0, A1, A0_adj, A1_adj  [N][num_lm][C]
//                   M0, H1, M0_adj, H1_adj  [N][num_LM][C]
//                   Phi1, dPhi1             [N][num_lme][C]
//   edge geometry   xyz [E][3] f64, r [E] f64
//   directed forces f   [E][3] f64
//   H1 messages     msg [E][num_LM][C] (H1-adjoint contributions per edge)
//   spline tables   R0 folded per ordered active pair:
//                     [pair_o][interval][l_max+1][C][4]
//                   R1 per unordered active pair:
//                     [pair_u][interval][num_paths][C][4]
//                   (the 4 cubic coefficients of one channel are one 16-byte
//                   load; a wave reads 1 KiB contiguous per path)
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sxl {

// Work this library issues on the calling thread: kernel launches (every
// launch site calls note_launch() after its <<<...>>>), device allocations
// and host waits on a stream.  Counted per thread, so that the counts an
// evaluator reads around one of its calls are its own while other threads
// drive other evaluators.
struct ThreadCounters {
    std::uint64_t launches = 0;
    std::uint64_t allocations = 0;
    std::uint64_t fences = 0;
};
ThreadCounters& thread_counters();
inline void note_launch() { ++thread_counters().launches; }
// hipStreamSynchronize, counted as one host fence.
inline hipError_t host_fence(hipStream_t s)
{
    ++thread_counters().fences;
    return hipStreamSynchronize(s);
}

struct EdgeGraph {
    int num_nodes = 0;
    int num_edges = 0;
    const int* node_types = nullptr;   // [N] model element index
    const int* type_active = nullptr;  // [num_elements] active index or -1
    int num_active = 0;
    const int* first = nullptr;        // [N+1] receiver offsets
    const int* receiver = nullptr;     // [E]
    const int* source = nullptr;       // [E]
    const int* tfirst = nullptr;       // [N+1] source-major offsets
    const int* tedge = nullptr;        // [E] edge ids grouped by source, ascending
    const int* edge_pair = nullptr;    // [E] ordered pair | unordered-pair table << 16 (active types; table 0 when shared)
    const double* xyz = nullptr;       // [E][3]
    const double* r = nullptr;         // [E]
    // The per-edge arrays (edge_pair, xyz, r, and the directed forces and
    // messages the kernels write) hold edge e at index e - edge_base.  The
    // untiled plan passes graph-wide arrays (edge_base 0, edge ids below
    // 2^31); the tiled plan passes tile-local receiver offsets, every
    // graph-wide edge array from the tile's first edge on and the tile's
    // source-grouped list as tedge, so edge ids are tile-local and edge_base
    // is 0 there too.
    long long edge_base = 0;
};

struct SplineGrid {
    double x0 = 0.0;
    double h = 0.0;
    int intervals = 0;  // knots - 1
    double r_cut = 0.0;
};

// Symmetric-contraction polynomial of one model (M0 or the M1 readout
// polynomial): the terms matched to a compiled monomial table (poly_shapes.inc,
// selected by `core` = its correlation order, 0 = none) occupy the first
// slots of each type's coefficient block, the remaining terms follow and run
// in a runtime loop.
struct PolyArgs {
    int core = 0;                      // correlation order of the compiled table, 0 = none
    int stride = 0;                    // coefficient slots per active type
    int num_rem = 0;                   // remainder terms
    const int* rem_offsets = nullptr;  // [outputs+1] remainder terms grouped by output
    const int* rem_packed = nullptr;   // [num_rem] deg | i0<<4 | i1<<10 | i2<<16
    const float* coef = nullptr;       // [active_type][stride][C] floats: compiled slots first, then the
                                       // remainder slots [slot][C]; the M0 table holds its compiled slots
                                       // in runs of four per channel ([slot / 4][C][4], padded to a
                                       // multiple of four slots), the readout table [slot][C]
};

// Slots of the compiled terms of an M0 coefficient block: the term count
// padded to whole runs of four.
constexpr int compiled_slots(int terms) { return (terms + 3) / 4 * 4; }

// Nodes grouped by active type: each block holds up to a fixed number of
// nodes of one type, so that a thread applies each coefficient it loads to
// several nodes.  A launch covers blocks [first, first + count).
struct NodeBlock {
    int start;  // first index into order
    int count;  // nodes in the block
    int type;   // active type index
    int pad;
};
struct NodeBlocks {
    const int* order = nullptr;         // node ids grouped by (tile, active type), ascending within
    const NodeBlock* blocks = nullptr;
    int first = 0;
    int count = 0;
    int block_nodes = 0;  // most nodes in one block of the list
};
constexpr int kM0BlockNodes = 4;       // nodes per block of the M0 kernels
// nodes per block of the M0 forward on launches that fill the machine twice
// over even so (the readout's rule): each coefficient load serves eight nodes
// (two waves per SIMD at 210-250 VGPRs; measured: water 0.45 -> 0.33 ms,
// 20,000 atoms 80 -> 74 us; 5,000 atoms 23.6 -> 26.0 us, hence four there)
constexpr int kM0ForwardBlockNodesWide = 8;
// nodes per block of the M0 reverse at C <= 128 when the launch is small:
// its blocks are two waves of 200 VGPRs, and four nodes per block leave a
// 5,000-atom launch one and a fraction waves per SIMD (measured: 66 -> 55 us
// at two nodes per block; 20,000 atoms: unchanged; C = 256: slower)
constexpr int kM0ReverseBlockNodesNarrow = 2;
constexpr int kReadoutBlockNodes = 8;  // nodes per block of the readout kernel
// nodes per readout block at C <= 128 when the launch is small: eight per
// block leave a 5,000-atom launch 625 workgroups of two waves (measured:
// 83 -> 77 us at two per block; 20,000 atoms: 242 -> 252 us; C = 256 on
// water: 0.77 -> 0.97 ms)
constexpr int kReadoutBlockNodesNarrow = 2;

struct GemmRows {
    const float* ptr = nullptr;
    long long node_stride = 0;  // floats between consecutive nodes
    long long row_stride = 0;   // floats between consecutive rows of one node
};

struct GemmOut {
    float* ptr = nullptr;
    long long node_stride = 0;
    long long row_stride = 0;
};

// Optional per-element-type bias of a GEMM's output rows:
// bias(node, m)[n] = ptr[node_types[node_base + node] * type_stride + m * row_stride + n]
struct GemmBias {
    const float* ptr = nullptr;
    const int* node_types = nullptr;  // element type of each graph node
    int node_base = 0;                // graph index of the GEMM's node 0
    long long type_stride = 0;
    long long row_stride = 0;
};

// out(node, m)[n] (+)= sum_k in(node, m)[k] Bt[n][k] + bias(node, m)[n]
// (Bt: Ncols x K row-major, i.e. the right-hand matrix transposed, so both
// operands are K-contiguous; accumulate adds to what out holds)
struct GemmArgs {
    int nodes = 0;
    int rows_per_node = 0;
    int K = 0;      // multiple of 32
    int Ncols = 0;
    GemmRows a;
    const float* Bt = nullptr;
    GemmOut c;
    GemmBias bias;
    int accumulate = 0;
    // GEMM node n is graph node node_ids[n] for the input and output rows
    // (null: node n); the bias is not remapped
    const int* node_ids = nullptr;
};

// Up to kMaxGemmGroup independent GEMMs (the irrep blocks of one stage) in
// one launch; tile_start is filled by the launcher.
constexpr int kMaxGemmGroup = 9;
struct GemmGroup {
    int count = 0;
    GemmArgs g[kMaxGemmGroup];
    int tile_start[kMaxGemmGroup + 1] = {};
};
hipError_t launch_gemm_group(GemmGroup group, hipStream_t stream);

// Density normalisation of A0 or A1 (reference compute/reverse_A0_scaled,
// mace.cpp:1561-1636, 2380-2458): per receiver s = 1 + sum over all its
// neighbours of a scalar spline f_pair(r); the features are divided by s and
// the reverse adds (adj . feature) / s * f'(r) r_hat to every directed force.
struct DensityScale {
    const float* table = nullptr;  // [pair_u][interval][4] cubic coefficients; null: no scaling
    float* scale = nullptr;        // [N] s per node (A1: written by the R1 forward)
    float* dot = nullptr;          // [N] adjoint . feature per node (A1: written by the readout)
};

struct LayerArgs {
    EdgeGraph graph;
    SplineGrid grid;
    DensityScale d0, d1;  // A0 and A1 density normalisation
    int C = 0;
    int l_max = 0, L_max = 0;
    int node_offset = 0;  // first receiver handled by this launch
    int node_count = 0;   // receivers handled by this launch
    // Receiver-indexed work arrays (A0, M0, Phi1, their adjoints) hold rows
    // i - local_base: 0 when the arrays span the whole graph, the tile's
    // first receiver in tiled execution (per-edge arrays: graph.edge_base).
    int local_base = 0;
    // receivers of this launch in element-type order (layer-0 kernels), or null
    const int* type_order = nullptr;
    // Second-interaction forward: workgroups per receiver, each over a slice
    // of 64 channels with its 4 waves splitting the edges (1: one workgroup
    // of all channels).  Set where the coefficient table outgrows one XCD's
    // L2: each XCD then reads only its slice's columns.
    int channel_slices = 1;
    // Layer-0 forward: workgroups per receiver, each over a slice of 64
    // channels with its 4 waves splitting the edges (1: one workgroup of all
    // channels); set for graphs whose receivers leave SIMDs idle.
    int a0_slices = 1;
    // Second-interaction reverse: one-wave workgroups per (receiver,
    // 64-channel slice), block b on XCD b mod 8 running slice
    // b mod reverse_slices (1: one workgroup of all channels).
    int reverse_slices = 1;
    // Edge-tile launches of the unsliced R1 reverse and the A0 reverse (their
    // per-receiver state is read-only and their outputs are per edge): one
    // workgroup per (receiver, first edge) entry, the receiver's edges from
    // there for at most edge_tile edges (16, 32 or kEdgeTile = 64), entries
    // in receiver order (edge_tiles) or in the layer-0 receiver order
    // (edge_tiles_layer0).  Null: one workgroup per receiver over all its
    // edges.  Each edge's force and message are reduced over the channels
    // alone, whichever tile holds it, so the results are the same bit for bit.
    const int* edge_tiles = nullptr;         // [num_edge_tiles][2]
    const int* edge_tiles_layer0 = nullptr;  // [num_edge_tiles][2]
    int num_edge_tiles = 0;
    int edge_tile = 64;
    // Layer 0 with the unfolded table: rows per unordered pair table (no H0,
    // no A0_W); each edge's radial values are scaled by
    // h0[source's active type][k] and A0_W is applied to the node sums by
    // GEMMs.  Null: the table folds H0 and A0_W per ordered pair.
    const float* h0 = nullptr;  // [active types][C]
};

// Layer 0: A0[i] = sum_j R0f_{pair(i,j)}(r) Y(r_hat)   (H0 and A0_W folded in),
// divided by the A0 density scale when the model has one; with a.h0 the
// table is the unfolded one and A0 holds the sums before A0_W
hipError_t launch_a0_forward(const LayerArgs& a, const float* r0f, float* A0, hipStream_t s);
// M0 = P0(A0) per (node, LM, channel), over the nodes of the given blocks
hipError_t launch_m0_forward(const LayerArgs& a, const PolyArgs& p0, const NodeBlocks& nb, const float* A0,
                             float* M0, hipStream_t s);
// Layer 1 forward: Phi1[i] = sum_j sum_terms cg R1 Y H1[src]
hipError_t launch_r1_forward(const LayerArgs& a, const float* r1, const float* cg, const float* H1,
                             float* Phi1, hipStream_t s);

struct ReadoutArgs {
    NodeBlocks nodes;               // nodes of this launch (readout block size)
    int local_base = 0;             // A1 / A1_adj hold rows i - local_base
    long long m0_stride = 0;        // floats between the M0 scalar rows of consecutive nodes
    int C = 0;
    int num_lm = 0;
    int num_LM = 0;
    int hidden = 0;
    const int* node_types = nullptr;
    const int* type_active = nullptr;
    const float* A1 = nullptr;      // [N][num_lm][C]
    const float* a1_scale = nullptr;  // [N] A1 density scale per node, null: unscaled model
    float* a1_dot = nullptr;          // [N] A1_adj . A1 per node (scaled model)
    const float* M0 = nullptr;      // scalar block (LM 0) of node i at M0 + i * m0_stride
    PolyArgs p1;
    // the H2 weights in runs of four of the streamed index per lane index
    // (runs4: [in / 4][out][4] for a matrix read as [in][out])
    const float* H2M0 = nullptr;    // [active] runs4 of [in][out]
    const float* H2M0T = nullptr;   // [active] runs4 of [out][in]
    const float* H2M1 = nullptr;    // runs4 of [in][out]
    const float* H2M1T = nullptr;   // runs4 of [out][in]
    const float* q = nullptr;       // [C]
    const float* W1 = nullptr;      // [hidden][C]
    const float* W2 = nullptr;      // [hidden]
    float scale = 1.0f;
    const double* E0 = nullptr;     // [active]
    double* energies = nullptr;     // [N]
    float* direct = nullptr;        // [N][C]
    float* A1_adj = nullptr;        // [N][num_lm][C]
};
hipError_t launch_readout(const ReadoutArgs& a, hipStream_t s);

constexpr int kEdgeTile = 64;     // edges per tile of the edge kernels
constexpr int kMinEdgeTile = 16;  // smallest edge tile of a tile-list launch

// Layer 1 reverse: directed forces (stored) and per-edge H1-adjoint messages.
// With reverse_slices > 1 (the (3, 2) shape, C = 64 x slices) each slice's
// part of the directed forces goes to `part` ([edges][slices][3] doubles,
// indexed like `forces`) before they are added in slice order; otherwise
// `part` is not read and may be null.
inline bool r1_reverse_sliceable(int l_max, int L_max, int C, int slices)
{
    return slices == 1 || (l_max == 3 && L_max == 2 && (slices == 2 || slices == 4) && C == 64 * slices);
}
hipError_t launch_r1_reverse(const LayerArgs& a, const float* r1, const float* cg, const float* H1,
                             const float* dPhi1, double* forces, float* msg, double* part, hipStream_t s);
// H1_adj[s] = sum over edges with source s of msg[e]
hipError_t launch_gather_messages(const LayerArgs& a, const float* msg, float* H1_adj,
                                  hipStream_t s);

// Tiled execution: the edges of one receiver tile grouped by source.  A run
// is (source, first index into the source-major edge list, length): the
// source's edges whose receivers lie in the tile.  H1_adj[source] += the
// run's messages (tile-local rows e - graph.edge_base), run by run.
struct TileRuns {
    int count = 0;
    const int* source = nullptr;
    const int* start = nullptr;   // into graph.tedge: the tile's source-grouped edge list
    const int* length = nullptr;
};
// Source-grouped edge list of one receiver tile (built once per graph, tile
// by tile in order): sources [E_t] are the tile's edge sources (tile-local
// edge l at index l).  mark: each source seen for the first time in this
// tile (last_tile [N] holds an earlier tile for it) becomes a run --
// run_source[k] = source, run_of[source] = k (k from *run_count, which
// starts at 0); lengths: run_length[run_of[source]] += 1 per edge (zeroed
// first); fill: list[run_start[k] + j] = the tile-local edge ids of run k
// (cursors zeroed first), in any order -- a segment sort makes them
// ascending.  mark with run_source null only counts the runs.
hipError_t launch_tile_runs_mark(int tile_edges, const int* sources, int tile, int* last_tile, int* run_of,
                                 int* run_source, int* run_count, hipStream_t s);
hipError_t launch_tile_runs_length(int tile_edges, const int* sources, const int* run_of, int* run_length,
                                   hipStream_t s);
hipError_t launch_tile_list_fill(int tile_edges, const int* sources, const int* run_of, const int* run_start,
                                 int* cursors, int* list, hipStream_t s);
hipError_t launch_fill_i32(int* out, long long n, int value, hipStream_t s);

// A caller's neighbour arrays checked on the device: flags[0] += edges whose
// source is outside [0, num_nodes), [1] whose type is outside the model,
// [2] whose type is not active, [3] whose type differs from the source's.
hipError_t launch_check_neighbors(long long num_edges, int num_nodes, const int* source, const int* neigh_types,
                                  const int* node_types, const int* type_active, int num_elements,
                                  unsigned long long* flags, hipStream_t s);

// A LAMMPS KOKKOS full neighbour list in device memory (the pair style's
// d_ilist, d_numneigh, d_neighbors, x, type; local_of[j] =
// atom->map(atom->tag[j]) filled by the caller; mace_types a device copy of
// the pair_coeff map): neighbour slot jj of atom i at neighbors[i stride_atom
// + jj stride_slot], masked with NEIGHMASK.
constexpr int kNeighMaskDevice = 0x1FFFFFFF;
struct PairList {
    int inum = 0;
    const int* ilist = nullptr;
    const int* numneigh = nullptr;
    const int* neighbors = nullptr;
    long long stride_atom = 0, stride_slot = 0;
    int nall = 0;
    const double* x = nullptr;
    const int* type = nullptr;
    const int* local_of = nullptr;
    int ntypes = 0;
    const int* mace_types = nullptr;
    double r_cut_squared = 0.0;
    // Stable topology (the reference's prepared execution): every listed
    // neighbour becomes an edge; one at r >= r_cut is scaled to length r_cut
    // (inactive in every edge kernel).  With neigh_indices null the fill pass
    // writes only xyz and r (a geometry update of an unchanged list) and flags
    // 16 when an entry's neighbour count differs from its offsets.
    int stable = 0;
    double r_cut = 0.0;
};
// ii_from_i [nall] (filled with -1 first): ilist position of each listed atom
hipError_t launch_pair_index(int inum, const int* ilist, int nall, int* ii_from_i, unsigned* flags, hipStream_t s);
// count pass (offsets null): node_types and counts of neighbours within r_cut
// (stable: of every listed neighbour) per list entry, flags (bits: 1 ilist,
// 2 neighbour index, 4 type, 8 local atom outside ilist); fill pass: the
// edges at offsets, in list order
hipError_t launch_pair_edges(const PairList& p, const int* ii_from_i, const long long* offsets, int* node_types,
                             int* counts, int* neigh_indices, int* neigh_types, double* xyz, double* r, unsigned* flags,
                             hipStream_t s);
// f[ilist[ii]] += node_forces[ii]; eatom[ilist[ii]] = node_energies[ii] (eatom may be null)
hipError_t launch_pair_scatter(int inum, const int* ilist, const double* node_forces, const double* node_energies,
                               double* f, double* eatom, hipStream_t s);
hipError_t launch_gather_tile_runs(const LayerArgs& a, const TileRuns& runs, const float* msg,
                                   float* H1_adj, hipStream_t s);
// M0_adj[:, LM 0, :] += direct
hipError_t launch_add_direct(int nodes, int C, int num_LM, const float* direct, float* M0_adj,
                             hipStream_t s);
// A0_adj = sum_LM M0_adj[LM] dP0_LM/dA0, over the nodes of the given blocks
hipError_t launch_m0_reverse(const LayerArgs& a, const PolyArgs& p0, const NodeBlocks& nb, const float* A0,
                             const float* M0_adj, float* A0_adj, hipStream_t s);
// Layer 0 reverse: forces += -(dE/dxyz) through R0f and Y (A0: the scaled
// features, used by the density-scale reverse)
hipError_t launch_a0_reverse(const LayerArgs& a, const float* r0f, const float* A0, const float* A0_adj,
                             double* forces, hipStream_t s);

// ZBL pair repulsion (zbl_kokkos.cpp:76-201), in double: energies[i] +=
// sum over all neighbours of V, forces[e] -= r_hat dV/dr.  Per ordered active
// pair: 1/a, 14.3996 Zu Zv, r_max = cov(Zu) + cov(Zv).
struct ZblArgs {
    const double* inverse_a = nullptr;
    const double* prefactor = nullptr;
    const double* r_max = nullptr;
    double c[4] = {};
    int p = 0;
};
// ZBL of receivers [node_begin, node_begin + num_nodes); the per-edge arrays
// hold edge e at index e - edge_base
hipError_t launch_zbl(int node_begin, int num_nodes, const int* first, long long edge_base, const int* edge_pair,
                      const double* xyz, const double* r, const ZblArgs& z, double* energies, double* forces,
                      hipStream_t s);

// Reference geometry of a prepared graph (reference
// prepare_factorized_geometry / _fractional_geometry / _shift_geometry,
// mace_kokkos_factorized_lifecycle.cpp:2455-2733): an edge's current vector
// is its reference vector plus disp[src] - disp[recv], disp being each atom's
// displacement from its reference position, wrapped to the minimum image
// along the periodic axes.  Reference edge vectors are given directly
// (`edges`, fractional or Cartesian) or as integer cell shifts:
// pos_ref[src] - pos_ref[recv] + shift . cell (Cartesian positions).
struct GeometryRef {
    const double* positions = nullptr;  // [N][3] reference positions (fractional coordinates when fractional)
    const double* edges = nullptr;      // [E][3] reference edge vectors (fractional when fractional), or null
    const int* shifts = nullptr;        // [E][3] integer cell shifts when edges is null, or
    const signed char* shifts8 = nullptr;  // [E][3] the same in int8
    int fractional = 0;
    // fractional positions and shifts of a graph built on the device: the
    // edge vector is formed as the build formed its fractional edge vector
    // (from the positions wrapped to [0, 1) and the image), bit for bit
    int built = 0;
    int pbc = 7;                        // bit a set: lattice axis a is periodic
};

// Geometry from positions (reference prepared_edge_geometry,
// mace_kokkos_factorized_lifecycle.cpp:3024-3074): xyz = reference edge
// vector + disp[src] - disp[recv]; an edge of zero or non-finite length is
// set to (r_cut, 0, 0) (inactive) and counted in *invalid.
hipError_t launch_edge_geometry(int num_edges, const int* receiver, const int* source, const GeometryRef& ref,
                                const double* displacements, const double* cell, double r_cut, double* xyz, double* r,
                                unsigned long long* invalid, hipStream_t s);

// Tiled execution: the edges of receivers [node_begin, node_begin +
// node_count) in the tile arena (edge e at index e - edge_base): xyz, r and
// the pair code, from the prepared geometry (ref) and the atoms'
// displacements; edges of zero or non-finite length are set to (r_cut, 0, 0)
// and counted in *invalid (when given).  With in_arena the caller's edge
// vectors and lengths are already in the arena and only the pair codes are
// formed.  Pair codes come from pair_source (a graph-wide table) or from the
// active types of receiver and source.  The tiled plan passes every edge
// array from the tile's first edge on and tile-local receiver offsets, so
// edge_base is 0 and no index exceeds the tile.
struct TileGeometry {
    int node_begin = 0, node_count = 0;
    long long edge_base = 0;
    const int* first = nullptr;
    const int* source = nullptr;
    const int* node_types = nullptr;
    const int* type_active = nullptr;
    int num_active = 0;
    bool shared_tables = false;
    const int* pair_source = nullptr;
    GeometryRef ref;
    const double* disp = nullptr;
    const double* cell = nullptr;  // 9 doubles on the device
    bool in_arena = false;
    double r_cut = 0.0;
    double* xyz = nullptr;
    double* r = nullptr;
    int* edge_pair = nullptr;
    unsigned long long* invalid = nullptr;
};
hipError_t launch_tile_geometry(const TileGeometry& g, hipStream_t s);
// atom_forces[i] -= sum of the directed forces of receiver i's edges, for the
// tile's receivers, then atom_forces[source] += sum over each source run of
// the tile (deterministic order; forces hold edge e at index e - edge_base)
hipError_t launch_fold_tile_forces(int node_begin, int node_count, const int* first, const TileRuns& runs,
                                   const int* tedge, long long edge_base, const double* forces, double* atom_forces,
                                   hipStream_t s);
hipError_t launch_fill_f64(double* out, long long n, double value, hipStream_t s);

// Reductions (deterministic, f64)
hipError_t launch_atom_forces(int num_nodes, const int* first, const int* tfirst, const int* tedge,
                              const double* forces, double* atom_forces, hipStream_t s);
// partial sums per block then one final pass: out[0] = sum energies, out[1..9] = stress
// (accumulate: out += the totals instead of out =)
hipError_t launch_reduce_totals(int num_nodes, int num_edges, const double* energies,
                                const double* forces, const double* xyz, double inv_volume,
                                double* partials, int num_partials, double* out, hipStream_t s,
                                bool accumulate = false);
int reduce_totals_partials(int num_nodes, int num_edges);

// Neighbour graph construction (bit-identical to the reference's device
// algorithm); see neighbor.hip.
struct NeighborPlan {
    int num_nodes = 0;
    int bins[3] = {1, 1, 1};
    int reach[3] = {1, 1, 1};
    double cell[9] = {};
    double inverse_cell[9] = {};
    double cutoff_squared = 0.0;
};
hipError_t launch_neighbor_bins(const NeighborPlan& p, const double* positions, double* reference_fractional,
                                double* wrapped_positions, double* wrapped_fractional, int* wrap_shifts,
                                int* atom_bins, int* bin_sizes, hipStream_t s);
hipError_t launch_neighbor_fill_bins(const NeighborPlan& p, const int* atom_bins,
                                     const int* bin_offsets, int* bin_cursors, int* bin_atoms,
                                     hipStream_t s);
// Outputs of the neighbour search.  Count pass (offsets null): edges per
// receiver, the largest |cell shift| component over the edges (atomicMax,
// may be null) and, with last_tile ([N], -1 or an earlier tile for every
// source before the first launch of `tile`), the number of distinct sources
// the launch adds to the tile (atomicAdd into *tile_runs).  Fill pass: the
// sources, the cell shifts (int32, or int8 when shifts8 is set) and, when
// frac is set, the fractional edge vectors, at the receivers' offsets.
struct EdgeOutputs {
    const long long* offsets = nullptr;
    long long* counts = nullptr;
    int* max_shift = nullptr;
    int* last_tile = nullptr;
    int tile = 0;
    int* tile_runs = nullptr;
    int* sources = nullptr;
    int* shifts = nullptr;
    signed char* shifts8 = nullptr;
    double* frac = nullptr;
};
// receivers [receiver_begin, receiver_begin + receiver_count)
hipError_t launch_neighbor_edges(const NeighborPlan& p, const double* wrapped_positions,
                                 const double* wrapped_fractional, const int* wrap_shifts,
                                 const int* atom_bins, const int* bin_offsets, const int* bin_atoms,
                                 int receiver_begin, int receiver_count, const EdgeOutputs& out, hipStream_t s);

// Exclusive scans (int -> int64 offsets), scratch of scan_scratch_size() int64
std::size_t scan_scratch_size(int n);
hipError_t launch_exclusive_scan_i32(const int* in, int n, long long* out, long long* scratch,
                                     hipStream_t s);
hipError_t launch_exclusive_scan_i64(const long long* in, int n, long long* out, long long* scratch,
                                     hipStream_t s);
// int64 offsets -> int32 offsets and counts
hipError_t launch_narrow_offsets(const long long* offsets, int n, int* out_offsets, int* out_counts,
                                 hipStream_t s);
// receiver ids per edge, and the source-major transpose (deterministic order)
hipError_t launch_receivers(int num_nodes, const int* first, int* receiver, hipStream_t s);
hipError_t launch_transpose_count(int num_edges, const int* source, int* counts, hipStream_t s);
hipError_t launch_transpose_fill(int num_edges, const int* source, const int* tfirst, int* cursors,
                                 int* tedge, hipStream_t s);
hipError_t launch_sort_segments(int num_segments, const int* offsets, int* values, hipStream_t s);
// Velocity-Verlet updates of the device NVE driver (md.hip): x, v, f are
// [N][3] doubles, inv_m [N] (unit factor / mass), m [N] masses.
hipError_t launch_md_kick_drift(int num_atoms, double* x, double* v, const double* f, const double* inv_m,
                                double dtf, double dt, hipStream_t s);
// v += dtf f inv_m; with a gate, only when *gate <= gate_limit (device value)
hipError_t launch_md_kick(int num_atoms, double* v, const double* f, const double* inv_m, double dtf,
                          const double* gate, double gate_limit, hipStream_t s);
// out[0] = sum m |v|^2 over the atoms (deterministic two-stage sum)
int md_kinetic_partials(int num_atoms);
hipError_t launch_md_kinetic(int num_atoms, const double* v, const double* m, double* partials, int num_partials,
                             double* out, hipStream_t s);
// Displacements of the atoms from their reference positions (ref.positions,
// in the current cell when fractional), wrapped to the minimum image along
// the periodic axes of ref.pbc; out[0] = max |disp|^2, out[1] zeroed (the
// invalid-edge count of launch_edge_geometry).
hipError_t launch_atom_displacements(int n, const double* positions, const GeometryRef& ref, const double* cell,
                                     const double* inverse_cell, double* displacements, double* out, hipStream_t s);
// edge_pair[e] = ordered | unordered << 16 from the active indices of the
// receiver and source element types (unordered = 0 with shared tables)
hipError_t launch_edge_pairs(int num_edges, const int* receiver, const int* source,
                             const int* node_types, const int* type_active, int num_active,
                             bool shared_tables, int* edge_pair, hipStream_t s);

}  // namespace sxl
