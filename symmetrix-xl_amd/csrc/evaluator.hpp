// MI355X MACE evaluator: owns the device copy of a model and of one prepared
// graph, and runs the energy + force evaluation on one HIP stream.
//
// The public surface mirrors the reference evaluator's prepared-graph API
// (symmetrix/source/cpp/mace_kokkos.cpp:1561-1840, 2086-2203;
// libsymmetrix/source/mace_kokkos.hpp:339-460): prepare a graph and receive a
// generation token, set geometry (positions or edge vectors) for that token,
// evaluate, then read node energies, directed edge forces, reduced atom
// forces and the stress.  A stale token is rejected
// (mace_kokkos_evaluate.cpp:326-334).  One evaluator is not thread-safe.
#pragma once

#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "kernels.hpp"
#include "model.hpp"

namespace sxl {

class DeviceBuffer {
public:
    DeviceBuffer() = default;
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    ~DeviceBuffer();
    void reserve(std::size_t bytes);  // grow-only
    void release();
    void swap(DeviceBuffer& other) noexcept
    {
        std::swap(ptr_, other.ptr_);
        std::swap(bytes_, other.bytes_);
    }
    template <class T>
    T* as() const { return static_cast<T*>(ptr_); }
    std::size_t bytes() const { return bytes_; }

private:
    void* ptr_ = nullptr;
    std::size_t bytes_ = 0;
};

// Pinned (page-locked) host memory, grow-only: copies between it and the
// device are asynchronous DMA.
class PinnedBuffer {
public:
    PinnedBuffer() = default;
    PinnedBuffer(const PinnedBuffer&) = delete;
    PinnedBuffer& operator=(const PinnedBuffer&) = delete;
    ~PinnedBuffer();
    void reserve(std::size_t bytes);  // grow-only
    template <class T>
    T* as() const { return static_cast<T*>(ptr_); }

private:
    void* ptr_ = nullptr;
    std::size_t bytes_ = 0;
};

// Periodic neighbour graph on the device (reference
// build_periodic_neighbor_graph_kokkos, neighbor_graph_kokkos.cpp:38-405).
struct PeriodicGraph {
    int num_nodes = 0;
    long long num_edges = 0;
    DeviceBuffer first;           // [N+1] int (standalone builds)
    DeviceBuffer sources;         // [E] int
    DeviceBuffer shifts;          // [E][3] int, or int8 when shift_bytes == 1
    int shift_bytes = 4;
    DeviceBuffer fractional_xyz;  // [E][3] double (may be absent)
    DeviceBuffer fractional_positions;  // [N][3] double: positions . inverse_cell at the build
};

// Count pass of the periodic neighbour search: wrapped positions, sorted
// cell bins, per-receiver edge counts and their int64 offsets (device and
// host), the edge total, the largest |cell shift| component and, when
// tile_receivers > 0, the number of distinct edge sources of each receiver
// tile [t T, (t + 1) T).  The fill pass writes the edges from it.
struct PeriodicCount {
    NeighborPlan plan;
    DeviceBuffer wp, wf, wrap, atom_bins, bin_offsets, bin_atoms, offsets;
    long long num_edges = 0;
    int max_shift = 0;
    std::vector<long long> host_first;  // [N+1]
    int tile_receivers = 0;
    std::vector<int> tile_runs;         // [tiles]
};
void count_periodic_graph(const double* d_positions, int num_nodes, const double* cell, const double* inverse_cell,
                          double cutoff, hipStream_t stream, DeviceBuffer& fractional_positions, PeriodicCount& c,
                          int tile_receivers);
// sources [E] int; shifts [E][3] as int32 (shifts) or int8 (shifts8, when
// every component fits); fractional_xyz [E][3] when not null
void fill_periodic_graph(const PeriodicCount& c, hipStream_t stream, int* sources, int* shifts, signed char* shifts8,
                         double* fractional_xyz);

// Builds the graph of N positions (device pointer) with the given cell
// (int32 offsets and shifts, fractional edge vectors; at most 2^31 - 1 edges).
// Validates inputs like the reference and throws on failure.
void build_periodic_graph(const double* d_positions, int num_nodes, const double* cell,
                          const double* inverse_cell, double cutoff, hipStream_t stream,
                          PeriodicGraph& out);
void validate_periodic_inputs(int num_nodes, const double* cell, const double* inverse_cell,
                              double cutoff);
// Bins and stencil reach of the cell-binned search (validates like the
// reference, neighbor_graph_kokkos.cpp:38-166).
NeighborPlan neighbor_plan(int num_nodes, const double* cell, const double* inverse_cell, double cutoff);
int neighbor_plan_bins(const NeighborPlan& plan);

// Allocation-free variant of build_periodic_graph for callers that cannot
// allocate device memory: positions and outputs are the caller's device
// arrays (receiver_offsets [N+1], sources [capacity], shifts and
// fractional_xyz [capacity][3]); every intermediate array lives in one
// fixed device array of the library (graph.hip), which bounds the atoms and
// cell bins below.  *num_edges receives the edge count; when it exceeds
// edge_capacity a length error is thrown and only *num_edges is written.
// The work runs on `stream` and has completed on return.  Calls that overlap
// on one GPU share that array and race.
constexpr int kNoAllocMaxAtoms = 1 << 17;
constexpr int kNoAllocMaxBins = 1 << 18;
void build_periodic_graph_noalloc(const double* d_positions, int num_nodes, const double* cell,
                                  const double* inverse_cell, double cutoff, long long edge_capacity,
                                  int* d_receiver_offsets, int* d_sources, int* d_shifts, double* d_fractional_xyz,
                                  long long* num_edges, hipStream_t stream);
std::size_t noalloc_scratch_bytes();

// Placement of a symmetric-contraction polynomial's terms on the kernels'
// coefficient slots (see PolyArgs): JSON term j -> slot[j].
struct PolyLayout {
    int core = 0;        // correlation order of the compiled table used, 0 = none
    int core_terms = 0;  // compiled terms
    bool quad = false;   // compiled slots in runs of four per channel ([slot / 4][C][4])
    int stride = 0;      // slots per active type
    std::vector<int> slot;
    std::vector<int> rem_offsets;  // [outputs + 1]
    std::vector<int> rem_packed;
};
PolyLayout poly_layout(int input_lmax, int output_lmax, const std::vector<int>& offsets,
                       const std::vector<int>& degree, const std::vector<int>& index, bool quad);

// Bytes of device memory held by this library's buffers (all evaluators).
std::size_t device_bytes_in_use();

struct EvaluatorStats {
    int last_num_nodes = 0;
    long long last_num_edges = 0;
    int active_edges = 0;
    double last_evaluation_ms = 0.0;
    int graph_builds = 0;
    int evaluations = 0;
    int tiled_evaluations = 0;
    int tile_receivers = 0;  // receivers per tile of the prepared graph, 0 = untiled plan
    int num_tiles = 0;
    // Observability (reference mace_kokkos.cpp:925-970: prepared graph and
    // evaluation counts, preparation and evaluation fences): host time of
    // the last graph preparation; host waits on the stream summed over all
    // graph preparations and over all evaluations; kernel launches, device
    // allocations and host waits of the last evaluation.
    double last_graph_prepare_ms = 0.0;
    long long preparation_fences = 0;
    long long evaluation_fences = 0;
    long long last_evaluation_launches = 0;
    long long last_evaluation_allocations = 0;
    long long last_evaluation_fences = 0;
};

// Receivers per tile chosen by the planner when tiled execution is allowed
// and the untiled workspace does not fit (reference mace_kokkos.hpp:542).
constexpr int kDefaultTileReceivers = 32768;

// Coefficient-table size above which the second-interaction forward of a
// 256-channel model runs in 64-channel slices.  Measured: the wide shape's
// 17.8 MB table (C = 256, 4 slices) 9.4 -> 6.9 ms on 30,000 water atoms.  At
// C = 128 two slices lose whatever the table size: the medium shape's 5.2 MB
// table 0.31 -> 0.38 ms, its 31 MB per-pair (Agnesi) tables 0.33 -> 0.39 ms,
// the wide shape's 8.9 MB table at C = 128 3.2 -> 3.6 ms.
constexpr std::size_t kR1SliceTableBytes = std::size_t(8) << 20;
// The layer-0 table folds H0[source type] and A0_W[receiver type] per ordered
// pair of active types (no extra work per edge).  Past this size (many
// active types) the untiled plan uses the unfolded table instead -- one per
// unordered radial table, resident in L2 -- with H0 applied per edge and A0_W
// by per-type node GEMMs: the folded rows otherwise stream from HBM.
// Measured on 20,000-atom irregular boxes (full calls, medium model): 4
// types (33 MB folded) 6.64 ms folded / 6.88 unfolded, 6 types (75 MB)
// 6.97 / 6.97-7.04, 8 types (134 MB) 7.31-7.37 / 6.97-7.07.
constexpr std::size_t kA0FoldedTableBytes = std::size_t(100) << 20;

// Execution-plan report (reference execution_plan.hpp:32-50 and
// mace_kokkos_runtime.cpp:3843-3915): the candidate plans with their memory
// estimates for the prepared graph and the one selected.  Plan identifiers
// are the reference's: "mh0-direct-speed" (untiled: graph-wide work arrays
// and per-edge messages) and "mh0-dual-layer-tiled-v1" (receiver tiles with
// one reused arena).
struct PlanCandidate {
    std::string id;
    bool qualified = false;
    std::size_t estimated_bytes = 0;
    std::string reason;
};
struct ExecutionPlanReport {
    std::string requested_algorithm = "direct";
    std::string requested_profile = "capacity";
    std::string selection_source = "native_request";
    std::string state = "pending";
    std::string selected_id;
    std::string selection_reason = "awaiting a prepared graph";
    std::size_t available_bytes = 0;
    std::size_t reserve_bytes = 0;
    bool boundary_attempt = false;
    std::vector<PlanCandidate> candidates;
    std::string json() const;
};

// Stages of one evaluation, timed with HIP events on the evaluator's stream
// when profiling is enabled.
enum Stage {
    kStageGeometry = 0,
    kStageA0Forward,
    kStageM0Forward,
    kStageH1Gemm,
    kStageR1Forward,
    kStageA1Gemm,
    kStageReadout,
    kStageA1ReverseGemm,
    kStageR1Reverse,
    kStageGather,
    kStageH1ReverseGemm,
    kStageM0Reverse,
    kStageA0Reverse,
    kStageAtomForces,
    kNumStages
};
const char* stage_name(int stage);

class Evaluator {
public:
    Evaluator(const std::string& model_path, const std::string& head);
    ~Evaluator();

    const HostModel& model() const { return model_; }
    hipStream_t stream() const { return stream_; }

    // --- graphs -------------------------------------------------------------
    // Receiver-major CSR given by the caller (neighbour lists of the caller,
    // e.g. a LAMMPS full list): neigh_types are model element indices.
    std::uint64_t prepare_graph(int num_nodes, const int* node_types, const int* num_neigh,
                                const int* neigh_indices, const int* neigh_types);
    // The same with every array in device memory (reference
    // prepare_factorized_graph_device, mace_kokkos.hpp:387-392): the node
    // types and counts are read back, the neighbour arrays checked and kept
    // on the device.
    std::uint64_t prepare_graph_device(int num_nodes, const int* d_node_types, const int* d_num_neigh,
                                       const int* d_neigh_indices, const int* d_neigh_types);
    // Periodic graph built on the device with cutoff + skin.  Positions are
    // host or device pointers (device_positions).
    std::uint64_t prepare_periodic_graph(int num_nodes, const int* node_types, const double* positions,
                                         bool device_positions, const double* cell,
                                         const double* inverse_cell, double cutoff);
    void update_cell(std::uint64_t generation, const double* cell, const double* inverse_cell);
    // Reference geometry of the prepared graph for evaluations from positions
    // (reference prepare_factorized_geometry / _fractional_geometry /
    // _shift_geometry, mace_kokkos_factorized_lifecycle.cpp:2455-2733): the
    // positions [N][3] and edge vectors [E][3] at which the caller built its
    // graph (Cartesian, or fractional in a fully periodic cell), or the
    // positions and integer cell shifts [E][3] of its edges; pbc [3] marks the
    // periodic lattice axes.  Sizes are the arrays' element counts.  A graph
    // built on the device carries its own (fractional) geometry.
    void prepare_geometry(std::uint64_t generation, const double* reference_positions, std::size_t num_positions,
                          const double* reference_xyz, std::size_t num_xyz, const double* cell,
                          const double* inverse_cell, const int* pbc, bool fractional);
    void prepare_shift_geometry(std::uint64_t generation, const double* reference_positions,
                                std::size_t num_positions, const int* shifts, std::size_t num_shifts,
                                const double* cell, const double* inverse_cell, const int* pbc);
    // 32-bit cardinality and extent checks of a graph before it is prepared
    // (reference validate_graph_cardinality, mace_kokkos_runtime.cpp:199-260).
    void validate_graph_cardinality(std::uint64_t num_receivers, std::uint64_t num_feature_nodes,
                                    std::uint64_t num_edges) const;
    long long num_edges() const { return num_edges_; }
    int num_nodes() const { return num_nodes_; }
    std::uint64_t generation() const { return generation_; }
    // Copies of the prepared periodic graph (host pointers, may be null).
    void graph_arrays(std::uint64_t generation, int* num_neigh, int* receiver_offsets, int* sources,
                      int* shifts, double* fractional_xyz) const;

    // --- geometry + evaluation ----------------------------------------------
    void compute_positions(std::uint64_t generation, const double* positions, bool device_positions);
    void compute_xyz(std::uint64_t generation, const double* xyz, const double* r, bool device_arrays);
    // Largest displacement (Angstrom) of positions from those of the last
    // periodic graph build, on the device (for neighbour-list skin reuse).
    double max_displacement(std::uint64_t generation, const double* positions, bool device_positions);
    double max_displacement_squared(std::uint64_t generation, const double* positions, bool device_positions);

    // --- device NVE molecular dynamics -----------------------------------------
    // Velocity-Verlet NVE run of `steps` steps of dt (fs) with positions,
    // velocities and forces resident on the device: x [N][3] (A) and v [N][3]
    // (A/fs) host arrays in/out, masses [N] (amu), epot / ekin [steps + 1]
    // (eV) and step_seconds [steps] (wall time of each step, the step's work
    // completed) host outputs (may be null).  The graph is built at r_cut +
    // skin and rebuilt on the device when an atom has moved more than skin/2.
    // Returns the number of rebuilds after the first build.
    int md_nve(int num_atoms, const int* node_types, const double* masses, double* x, double* v,
               const double* cell, const double* inverse_cell, double skin, double dt, int steps, double* epot,
               double* ekin, double* step_seconds);
    // Called on the host after each MD step (1-based) with its potential and
    // kinetic energy (NaN when not computed) and wall time; a nonzero return
    // stops the run after that step.  Null: none.
    using StepCallback = int (*)(int step, double epot, double ekin, double seconds, void* user);
    void set_md_progress(StepCallback callback, void* user)
    {
        md_progress_ = callback;
        md_progress_user_ = user;
    }

    // --- results -------------------------------------------------------------
    void node_energies(double* out) const;            // [N]
    void node_forces(double* out) const;              // [E][3] directed, -dE/dxyz
    void atom_forces(std::uint64_t generation, double* out);              // [N][3]
    void stress(std::uint64_t generation, double volume, double* out9);   // 3x3 row-major
    double total_energy(std::uint64_t generation);
    // device pointers of the results (valid until the next call)
    const double* device_atom_forces() const { return atom_forces_.as<double>(); }
    const double* device_node_energies() const { return energies_.as<double>(); }
    const double* device_totals() const { return totals_.as<double>(); }
    void synchronize() const;

    const EvaluatorStats& stats() const { return stats_; }

    // --- execution plan --------------------------------------------------------
    // Tiled ("fixed workspace") execution: receivers are processed in tiles
    // with a reused per-tile arena; graph-wide state is H1, its adjoint, the
    // scalar M0 block and the direct adjoint.  Both setters invalidate the
    // prepared graph (reference mace_kokkos_runtime.cpp:2771-2781, 3992-4000).
    void set_allow_fixed_workspace(bool allow);
    bool allow_fixed_workspace() const { return allow_fixed_workspace_; }
    void set_workspace_receiver_limit(int receivers);
    int workspace_receiver_limit() const { return receiver_limit_; }
    // Plan request (reference _set_execution_plan_request): algorithm
    // "direct"; profile "capacity" (tiles when the untiled estimate exceeds
    // the memory budget and fixed workspace is allowed) or "speed" (untiled);
    // debug_plan "" or a plan identifier to pin.  Invalidates the graph.
    void set_execution_plan_request(const std::string& algorithm, const std::string& profile,
                                    const std::string& debug_plan);
    const ExecutionPlanReport& execution_plan_report() const { return plan_report_; }
    // Device bytes by role and the plan's capacities, as a JSON object (the
    // workspace and policy properties of the Python class are read from it).
    std::string workspace_json() const;

    // Per-stage device time (ms) accumulated over profiled evaluations.
    // Replay untiled evaluations from positions as one HIP graph launch
    // (captured on the first call for a graph generation, positions array
    // and cell; recaptured when one of them changes).  Off by default.
    void set_graph_replay(bool enable);
    bool graph_replay() const { return graph_replay_; }
    void set_profiling(bool enable);
    // profile only the stages whose bit is set in mask (bit i = stage i)
    void set_profiling_stages(unsigned mask);
    // Largest displacement (A) of the last evaluation from positions, from
    // the same pass (no extra device work): callers may evaluate first and
    // rebuild and evaluate again when it exceeds their skin rule.
    double last_max_displacement() const;
    void stage_times(double* ms, int* counts) const;

private:
    void check_generation(std::uint64_t generation) const;
    void prepare_active_types(const std::vector<int>& node_types);
    void upload_static_tables();
    void finish_graph(const std::vector<int>& host_pairs);
    std::vector<int> caller_pairs(const int* host_neigh_types, const int* host_sources);
    bool tiles_possible(int num_nodes) const;
    void allocate_workspace();
    // Execution plan of the graph being prepared from host_first_ and the
    // edge count (before its edges are written), then the tiled plan's
    // tile-local offsets, source-grouped lists and runs (after)
    void select_plan();
    void build_tile_lists();
    void count_tile_runs();
    void release_untiled_edge_state();
    void plan_node_blocks();
    NodeBlocks node_blocks(const DeviceBuffer& blocks, const std::vector<int>& offsets, int tile,
                           int block_nodes) const;
    void invalidate_graph();
    void evaluate();
    void evaluate_tiled();
    void gemm_h1(int nodes, int node_base, const float* in, long long in_stride, float* out, long long out_stride,
                 bool reverse, float* x_out, const char* what);
    void add_direct(int nodes, int node_base, float* M0adj, hipStream_t s);
    void gemm_a1(int nodes, const float* in, float* out, bool reverse, const char* what);
    // A0 = A0_pre A0_W[type] per l block (reverse: A0_pre_adj = A0_adj A0_W^T),
    // the untiled plan's nodes grouped by active type
    void gemm_a0(const float* in, float* out, bool reverse);
    bool a0_unfolded() const { return a0_unfold_ && tile_receivers_ == 0; }
    void reduce(double volume);
    // counts of the calling thread at the start of a preparation/evaluation
    struct CallStart {
        ThreadCounters counters = thread_counters();
        std::chrono::steady_clock::time_point time = std::chrono::steady_clock::now();
    };
    void account_preparation(const CallStart& start);
    // waits for the stream and drops the host copies of staged uploads
    void wait(const char* what);
    void account_evaluation(const CallStart& start);

    HostModel model_;
    hipStream_t stream_ = nullptr;
    EvaluatorStats stats_;

    // shape
    int C_ = 0, nlm_ = 0, nLM_ = 0, nlme_ = 0;
    std::vector<int> num_e_, lme_off_;

    // model tables on the device
    std::vector<int> active_types_;
    DeviceBuffer type_active_, r0f_, r1_, p0_coef_, p0_packed_, p0_offsets_, p1_coef_, p1_packed_,
        p1_offsets_, h2m0_, h2m0t_, e0_;
    DeviceBuffer h1w_, h1wt_, h2m1_, h2m1t_, q_, w1_, w2_, cg_;
    // pre_linear_up basis: P0 ([in][out]) and P0^T; residual tables [ne][num_LM][C]
    DeviceBuffer p0w_, p0wt_, residual_, residual_fused_;
    // unfolded layer-0 table [pair_u][iv][l][k][q], H0 of the active types
    // [active][C], A0_W per active type [active][l][k][k'] and transposed;
    // A0_pre: the layer-0 sums before A0_W [N][nlm][C]
    bool a0_unfold_ = false;
    DeviceBuffer r0u_, h0s_, a0w_, a0wt_, A0pre_;
    // host copies of both layer-0 tables of the active types; only the one
    // the selected plan reads is on the device (place_layer0_tables)
    std::vector<float> host_r0f_, host_r0u_, host_h0_, host_a0w_, host_a0wt_;
    void place_layer0_tables();
    std::vector<std::unique_ptr<DeviceBuffer>> a1w_, a1wt_;
    PolyLayout p0_layout_, p1_layout_;
    // density-normalisation splines [pair_u][interval][4] and ZBL pair tables [ordered active pair]
    DeviceBuffer dens0_, dens1_, zbl_inverse_a_, zbl_prefactor_, zbl_rmax_;
    PolyArgs poly_args(const PolyLayout& layout, const DeviceBuffer& coef, const DeviceBuffer& offsets,
                       const DeviceBuffer& packed) const;
    // The radial functions depend on the element pair only through a
    // distance transform with per-element radii; without one, every pair
    // shares one R1 and density table (table index 0 in edge_pair).
    bool shared_pair_tables() const { return !model_.agnesi; }
    SplineGrid grid_;

    // graph
    std::uint64_t generation_ = 0;
    std::uint64_t prepared_generation_ = 0;  // generation_ right after the last successful preparation
    std::uint64_t evaluated_generation_ = 0;
    bool periodic_ = false;
    int num_nodes_ = 0;
    long long num_edges_ = 0;
    std::vector<int> host_types_;
    std::vector<long long> host_first_;  // CSR receiver offsets of the prepared graph, [N + 1]
    // edges a graph may have under the untiled plan, whose edge ids are int32
    // (2^31 - 1; SXL_EDGE_INDEX_LIMIT lowers it, a test hook); the tiled plan
    // indexes edges per tile and has no such limit
    long long edge_index_limit_ = 2147483647LL;
    int r1_slices_ = 1;            // channel slices of the second-interaction forward
    int r1_graph_slices_ = 1;      // and for the prepared graph (small untiled graphs slice more)
    int r1_rev_slices_ = 1;        // and of its reverse
    // host copies of uploads in flight, released at the next wait()
    std::vector<std::vector<unsigned char>> staged_;
    double cell_[9] = {}, inverse_cell_[9] = {};
    PeriodicGraph pgraph_;
    // cell_dev_: cell (9) then inverse cell (9); disp_: [N][3] minimum-image
    // displacements from the build's fractional positions in the current cell.
    // Untiled plan: first_ [N+1] receiver offsets, tfirst_ / tedge_ the
    // source-major transpose.  Tiled plan: first_ holds tile-local offsets,
    // tile t's receivers at [t (T + 1), t (T + 1) + count] (so first_ + t
    // indexed by graph receiver ids), and tedge_ each tile's source-grouped
    // list of tile-local edge ids at its first edge (no tfirst_).
    DeviceBuffer node_types_, first_, receiver_, source_, tfirst_, tedge_, edge_pair_, disp_, positions_,
        cell_dev_;
    bool check_geometry_ = false;          // evaluation from positions: invalid edges raise
    unsigned long long invalid_edges_ = 0;
    void upload_cell();
    void finish_evaluation();
    void enqueue_evaluation();
    void enqueue_totals();
    void complete_evaluation();
    void after_evaluation(std::chrono::steady_clock::time_point t0);
    double cell_volume() const;
    // the geometry kernels of an evaluation from positions (src: device
    // positions, or positions_ after the staged host copy)
    void enqueue_positions(const double* src, bool device_positions);
    // HIP graph replay of untiled evaluations from positions: the kernels
    // from the positions copy to the totals are captured once per (graph
    // generation, positions array, cell) and replayed with one launch
    bool graph_replay_ = false;
    hipGraph_t replay_graph_ = nullptr;
    hipGraphExec_t replay_exec_ = nullptr;
    struct ReplayKey {
        std::uint64_t generation = 0;
        const double* positions = nullptr;
        bool device = false;
        double cell[9] = {};
        bool operator==(const ReplayKey& o) const;
    };
    ReplayKey replay_key_;
    long long replay_launches_ = 0;  // kernels in the captured graph
    void release_replay();
    DeviceBuffer xyz_, r_;
    // reference geometry for evaluations from positions (see prepare_geometry)
    enum GeometryMode { kGeometryNone = 0, kGeometryBuilt, kGeometryCartesian, kGeometryFractional, kGeometryShifts };
    GeometryMode geometry_mode_ = kGeometryNone;
    std::uint64_t geometry_generation_ = 0;
    int geometry_pbc_ = 7;
    DeviceBuffer geo_positions_, geo_edges_, geo_shifts_;
    GeometryRef geometry_ref() const;
    void require_geometry(std::uint64_t generation) const;
    void set_cell(const double* cell, const double* inverse_cell);

    // workspace
    DeviceBuffer A0_, M0_, H1_, Phi1_, A1_, A1adj_, direct_, H1adj_, msg_, rpart_, energies_, forces_,
        atom_forces_, partials_, totals_, scratch_;
    DeviceBuffer scale1_, dot1_;  // [N] A1 density scale and A1_adj . A1 (scaled models)
    void density_args(LayerArgs& la, ReadoutArgs* ra);
    void launch_zbl_term(const LayerArgs& la, double* forces, hipStream_t s);
    bool reduced_ = false;
    double reduced_volume_ = 0.0;
    // host copy of totals_: [0] energy, [1..9] stress 3x3, [12] max |disp|^2,
    // [13] invalid-edge count; an evaluation from positions reduces energy and
    // stress (cell volume) in the same pass and fills it with one copy
    double host_totals_[32] = {};
    // an evaluation from host positions also copies the node energies and
    // atom forces to pinned host memory before its one wait, so reading them
    // afterwards needs no device access (host_results_: they belong to the
    // current evaluation)
    PinnedBuffer pinned_positions_, pinned_energies_, pinned_forces_;
    bool results_to_host_ = false;
    bool host_results_ = false;
    void set_stress_from_virial(double volume);
    double fused_volume_ = 0.0;
    bool last_from_positions_ = false;

    // tiled plan
    bool allow_fixed_workspace_ = false;
    int receiver_limit_ = 0;
    std::string plan_profile_ = "capacity", plan_debug_;
    ExecutionPlanReport plan_report_;
    std::size_t graph_bytes_estimate(bool tiled, long long runs) const;
    std::size_t held_graph_bytes() const;
    std::size_t work_bytes_estimate(long long receivers, long long edges, bool tiled) const;
    // tile arena: geometry, pair codes and directed forces of one tile's
    // edges (edge e at index e - first edge of the tile)
    DeviceBuffer tile_xyz_, tile_r_, tile_pair_, tile_forces_;
    // pair codes follow from the node types of receiver and source (false when
    // a caller's neighbour types differ: the tiled plan then keeps edge_pair_)
    bool pair_from_types_ = true;
    // the last evaluation's edge vectors came from the caller rather than
    // from the prepared geometry; the tiled plan copies each tile's slice of
    // the caller's arrays (host or device, valid during that call) into the
    // arena instead of keeping them graph-wide
    bool explicit_geometry_ = false;
    const double* explicit_xyz_ = nullptr;
    const double* explicit_r_ = nullptr;
    bool explicit_device_ = false;
    // tiled plan: -sum_e f_e (x) xyz_e of the last evaluation (stress = this / V)
    double host_virial_[9] = {};
    int tile_receivers_ = 0;
    int num_tiles_ = 0;
    std::vector<long long> tile_first_edge_;  // [num_tiles + 1]
    std::vector<int> tile_run_offsets_;       // [num_tiles + 1]
    // distinct edge sources per tile of the graph being prepared (from the
    // count pass of a device build; empty: counted from the sources)
    std::vector<int> tile_runs_;
    // M0s_: [N][C] scalar readout input x (M0 scalar block, or M0_scalar P0
    // (+ residual) in the pre_linear_up basis), graph-wide
    DeviceBuffer M0s_, run_source_, run_start_, run_length_;
    // device NVE driver state: positions, velocities, masses, unit factor / mass, kinetic partials
    DeviceBuffer md_x_, md_v_, md_m_, md_inv_m_, md_partials_;
    // Work queued behind an evaluation from positions and before its one
    // host wait (the MD driver's kick and kinetic energy); null otherwise.
    std::function<void()> epilogue_;
    StepCallback md_progress_ = nullptr;
    void* md_progress_user_ = nullptr;
    // nodes grouped by (tile, active type) and their blocks for the node kernels
    DeviceBuffer node_order_, m0_blocks_, m0r_blocks_, readout_blocks_;
    // untiled plan: (receiver, first edge) of every 64-edge tile of the
    // receivers' edge lists, in receiver order and in the layer-0 order
    // (LayerArgs::edge_tiles); empty when SXL_EDGE_TILE_LAUNCH=0
    DeviceBuffer edge_tiles_, edge_tiles_l0_;
    int num_edge_tiles_ = 0;
    int edge_tile_ = kEdgeTile;  // edges per tile-list entry
    int a0_graph_slices_ = 1;    // layer-0 forward slices of the untiled plan (LayerArgs::a0_slices)
    // [tiles + 1] each; the M0 reverse has its own block size (m0r_block_nodes_)
    std::vector<int> m0_block_offsets_, m0r_block_offsets_, readout_block_offsets_;
    // untiled plan: each active type's nodes at node_order_[type_start_[a]
    // .. + type_count_[a])
    std::vector<int> type_start_, type_count_;
    int m0_block_nodes_ = kM0BlockNodes;
    int m0r_block_nodes_ = kM0BlockNodes;
    int readout_block_nodes_ = kReadoutBlockNodes;
    int compute_units_ = 0;  // of the evaluator's device

    bool profiling_ = false;
    unsigned profile_mask_ = 0;
    std::vector<hipEvent_t> events_;  // [stage][begin, end]
    double stage_ms_[kNumStages] = {};
    int stage_count_[kNumStages] = {};
    bool stage_used_[kNumStages] = {};
    void mark(int stage, bool end);
};

}  // namespace sxl
