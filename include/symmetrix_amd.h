/*
 * symmetrix_amd.h -- C ABI of the MI355X-native MACE evaluator.
 *
 * Drop-in boundary for the model-evaluation path of Symmetrix-XL: every entry
 * point below replaces one method of the reference's native evaluator class
 * MACEKokkosFloat, which the reference binds to Python with pybind11
 * (symmetrix/source/cpp/mace_kokkos.cpp) and calls from its ASE calculator
 * (symmetrix/source/symmetrix/calculator.py) and LAMMPS pair style
 * (pair_symmetrix/pair_symmetrix_mace.cpp).  The cited line of each function
 * is the reference interface it stands in for.
 *
 * Conventions (kept from the reference, mace_kokkos.hpp and
 * jit_host_plugin_abi.h:109-110):
 *   - plain pointers and sizes only; arrays are C-contiguous; host pointers
 *     unless a function name ends in _device;
 *   - node types are model element indices (not atomic numbers);
 *   - edges are receiver-major, contiguous per receiver; edge vector
 *     xyz = r_source - r_receiver (+ periodic shift . cell);
 *   - directed forces are f_e = -dE/dxyz_e (reference node_forces);
 *   - atom forces F_a = sum_{src=a} f_e - sum_{recv=a} f_e; stress
 *     sigma = -(1/V) sum_e f_e (x) xyz_e, row-major 3x3;
 *   - graph preparation returns a generation token; a stale token is an
 *     error (mace_kokkos_evaluate.cpp:326-334);
 *   - every function returns SXL_OK (0) or an error code and never throws;
 *     the message of the last error on the calling thread is sxl_last_error();
 *   - one evaluator owns one HIP stream and device memory and is not
 *     thread-safe; calls return after their device work has completed unless
 *     stated otherwise.
 */
#ifndef SYMMETRIX_AMD_H
#define SYMMETRIX_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SXL_OK 0
#define SXL_INVALID_ARGUMENT 1 /* std::invalid_argument in the reference  */
#define SXL_OUT_OF_RANGE 2     /* std::out_of_range                        */
#define SXL_LENGTH_ERROR 3     /* std::length_error (int32 cardinality)     */
#define SXL_RUNTIME_ERROR 4    /* std::runtime_error, device failures      */
#define SXL_LOGIC_ERROR 5      /* std::logic_error                          */
#define SXL_ALLOCATION_ERROR 6 /* host or device allocation failure         */

typedef struct sxl_evaluator sxl_evaluator;

typedef struct {
    int num_elements;
    int num_channels;
    int l_max;
    int L_max;
    int num_paths;
    int spline_points;
    double r_cut;
} sxl_model_info_t;

typedef struct {
    int64_t device_bytes;
    int num_nodes;
    int64_t num_edges;
    int graph_builds;
    int evaluations;
    double last_evaluation_ms; /* host time to enqueue and run one evaluation */
    int tiled_evaluations;     /* evaluations that ran the tiled plan */
    int tile_receivers;        /* receivers per tile of the prepared graph, 0 = untiled */
    int num_tiles;
    /* Observability counters (factorized_prepared_graph_count,
     * factorized_prepared_evaluation_count, factorized_preparation_fence_count,
     * factorized_evaluation_fence_count, mace_kokkos.cpp:925-970): host time
     * of the last graph preparation; host waits on the evaluator's stream
     * summed over graph preparations and over evaluations; kernel launches,
     * device allocations and host waits of the last evaluation. */
    double last_graph_prepare_ms;
    int64_t preparation_fences;
    int64_t evaluation_fences;
    int64_t last_evaluation_launches;
    int64_t last_evaluation_allocations;
    int64_t last_evaluation_fences;
} sxl_stats_t;

/* Message of the last failed call on this thread ("" if none). */
const char* sxl_last_error(void);

/* Load a format-4 compact MACE JSON for FP32 evaluation on the current HIP
 * device.  Replaces MACEKokkosFloat(filename, head)
 * (symmetrix/source/cpp/mace_kokkos.cpp:262-264). */
int sxl_create(const char* model_path, const char* head, sxl_evaluator** out);
void sxl_destroy(sxl_evaluator* evaluator);

/* Runtime lifecycle.  Replace the module functions _init_kokkos,
 * _finalize_kokkos, _kokkos_is_initialized, _kokkos_live_object_count and
 * _kokkos_default_execution_space (symmetrix/source/cpp/tools_kokkos.cpp:522-534;
 * libsymmetrix/source/tools_kokkos.cpp:44-99).  Creating an evaluator
 * initializes the runtime; finalization fails while evaluators are alive and
 * no evaluator can be created after it.  sxl_runtime_is_initialized returns
 * 1 or 0; sxl_default_execution_space returns "HIP". */
int sxl_runtime_initialize(void);
int sxl_runtime_finalize(void);
int sxl_runtime_is_initialized(void);
int64_t sxl_live_evaluator_count(void);
const char* sxl_default_execution_space(void);

/* Model metadata: r_cut, l_max, L_max, ... properties (mace_kokkos.cpp:2762). */
int sxl_model_info(const sxl_evaluator* evaluator, sxl_model_info_t* out);
/* atomic_numbers / atomic_energies properties: num_elements entries. */
int sxl_atomic_numbers(const sxl_evaluator* evaluator, int* out);
int sxl_atomic_energies(const sxl_evaluator* evaluator, double* out);

/* Receiver-major CSR from the caller.  Replaces
 * _prepare_factorized_graph(num_nodes, node_types, num_neigh, neigh_indices,
 * neigh_types) (mace_kokkos.cpp:1561-1579). */
int sxl_prepare_graph(sxl_evaluator* evaluator, int num_nodes, const int* node_types, const int* num_neigh,
                      const int* neigh_indices, const int* neigh_types, uint64_t* generation);
/* The same with the four arrays in device memory.  Replaces the C++
 * prepare_factorized_graph_device(num_nodes, node_types, num_neigh,
 * neigh_indices, neigh_types) over Kokkos views
 * (libsymmetrix/source/mace_kokkos.hpp:387-392): the node types and
 * neighbour counts are read back (2 N ints); the neighbour arrays are
 * checked and kept on the device. */
int sxl_prepare_graph_device(sxl_evaluator* evaluator, int num_nodes, const int* d_node_types,
                             const int* d_num_neigh, const int* d_neigh_indices, const int* d_neigh_types,
                             uint64_t* generation);

/* Periodic neighbour graph built on the device at `cutoff` (model cutoff plus
 * skin).  cell and inverse_cell are row-major 3x3 (rows are lattice vectors).
 * Replaces _prepare_periodic_factorized_graph(node_types, positions, cell,
 * inverse_cell, neighbor_cutoff) (mace_kokkos.cpp:1580-1603). */
int sxl_prepare_periodic_graph(sxl_evaluator* evaluator, int num_nodes, const int* node_types,
                               const double* positions, const double* cell, const double* inverse_cell,
                               double cutoff, uint64_t* generation, int64_t* num_edges);
int sxl_prepare_periodic_graph_device(sxl_evaluator* evaluator, int num_nodes, const int* node_types,
                                      const double* d_positions, const double* cell,
                                      const double* inverse_cell, double cutoff, uint64_t* generation,
                                      int64_t* num_edges);

/* Copies of the prepared periodic graph (any output may be NULL): num_neigh
 * [N], receiver_offsets [N+1], sources [E], shifts [E][3], fractional_xyz
 * [E][3].  Outputs of the reference's build_periodic_neighbor_graph_kokkos
 * (libsymmetrix/source/neighbor_graph_kokkos.cpp:38-405). */
int sxl_graph_arrays(sxl_evaluator* evaluator, uint64_t generation, int* num_neigh, int* receiver_offsets,
                     int* sources, int* shifts, double* fractional_xyz);

/* New cell for the prepared graph (_update_factorized_cell,
 * mace_kokkos.cpp:1673-1685): later evaluations form each edge vector as the
 * fractional reference edge vector (the device build's, or the caller's
 * fractional or shift geometry) in this cell plus the atoms' minimum-image
 * displacements.  Invalid argument without such a geometry, or when the cell
 * is non-finite, singular or (device-built graph) does not match its
 * inverse. */
int sxl_update_cell(sxl_evaluator* evaluator, uint64_t generation, const double* cell,
                    const double* inverse_cell);

/* 32-bit cardinality checks of a graph the caller is about to prepare:
 * length error when the receiver or feature-node count reaches INT32_MAX or
 * the edge count exceeds it, invalid argument when there are fewer feature
 * nodes than receivers.  Replaces _validate_graph_cardinality(num_receivers,
 * num_feature_nodes, num_edges) (symmetrix/source/cpp/mace_kokkos.cpp:1604-1607;
 * MACEKokkos::validate_graph_cardinality, mace_kokkos_runtime.cpp:199-260). */
int sxl_validate_graph_cardinality(const sxl_evaluator* evaluator, int64_t num_receivers, int64_t num_feature_nodes,
                                   int64_t num_edges);

/* Geometry of a graph prepared with sxl_prepare_graph, for evaluations from
 * positions (sxl_compute_prepared_positions*): the reference positions
 * [N][3] and the edge vectors [E][3] at which the caller built its graph, the
 * cell and its inverse (row-major 3x3) and pbc [3] (non-zero = periodic lattice
 * axis).  An evaluation at positions x forms each edge vector as the
 * reference edge vector + d[src] - d[recv], with d = x - reference position
 * wrapped to the minimum image along the periodic axes (no wrap without
 * one).  num_positions and num_xyz are element counts (3N, 3E); invalid
 * argument on a stale token, other extents or a non-finite value.  Replaces
 * _prepare_factorized_geometry(generation, reference_positions,
 * reference_xyz, cell, inverse_cell, pbc) (mace_kokkos.cpp:1608-1629). */
int sxl_prepare_geometry(sxl_evaluator* evaluator, uint64_t generation, const double* reference_positions,
                         int64_t num_positions, const double* reference_xyz, int64_t num_xyz, const double* cell,
                         const double* inverse_cell, const int* pbc);
/* As sxl_prepare_geometry with fractional reference positions and edge
 * vectors (in units of the lattice vectors), which follow later cells set by
 * sxl_update_cell; requires a fully periodic, invertible cell.  Replaces
 * _prepare_factorized_fractional_geometry(generation, fractional_positions,
 * fractional_xyz, cell, inverse_cell, pbc) (mace_kokkos.cpp:1650-1669). */
int sxl_prepare_fractional_geometry(sxl_evaluator* evaluator, uint64_t generation, const double* fractional_positions,
                                    int64_t num_positions, const double* fractional_xyz, int64_t num_xyz,
                                    const double* cell, const double* inverse_cell, const int* pbc);
/* As sxl_prepare_geometry with each reference edge vector given as
 * reference_position[src] - reference_position[recv] + shift . cell from
 * integer cell shifts [E][3] (12 bytes per edge); later cells set by
 * sxl_update_cell apply.  Replaces _prepare_factorized_shift_geometry(
 * generation, reference_positions, shifts, cell, inverse_cell, pbc)
 * (mace_kokkos.cpp:1630-1649), which the reference accepts only for its tiled
 * plans; here either plan. */
int sxl_prepare_shift_geometry(sxl_evaluator* evaluator, uint64_t generation, const double* reference_positions,
                               int64_t num_positions, const int* shifts, int64_t num_shifts, const double* cell,
                               const double* inverse_cell, const int* pbc);

/* Evaluate energies and forces at new positions of a prepared graph: a
 * periodic graph built on the device, or a caller's graph with a geometry set
 * by one of the functions above.  Replaces
 * _compute_prepared_factorized_positions(generation, positions)
 * (mace_kokkos.cpp:1828-1836).  Invalid argument when the graph has no
 * geometry, or when an edge of the graph has zero or non-finite length at
 * these positions (coincident atoms). */
int sxl_compute_prepared_positions(sxl_evaluator* evaluator, uint64_t generation, const double* positions);
int sxl_compute_prepared_positions_device(sxl_evaluator* evaluator, uint64_t generation,
                                          const double* d_positions);

/* Evaluate with caller-provided edge vectors xyz [E][3] and lengths r [E].
 * Replaces _compute_prepared_factorized(generation, xyz, r)
 * (mace_kokkos.cpp:1817-1827). */
int sxl_compute_prepared(sxl_evaluator* evaluator, uint64_t generation, const double* xyz, const double* r);
/* The same with xyz and r in device memory (the reference's C++
 * compute_prepared_factorized over device views, mace_kokkos.hpp:339-460);
 * they are read during the call only. */
int sxl_compute_prepared_device(sxl_evaluator* evaluator, uint64_t generation, const double* d_xyz,
                                const double* d_r);

/* One-shot: prepare the CSR graph and evaluate.  Replaces
 * compute_node_energies_forces(num_nodes, node_types, num_neigh,
 * neigh_indices, neigh_types, xyz, r) (mace_kokkos.cpp:2169-2203). */
int sxl_compute_node_energies_forces(sxl_evaluator* evaluator, int num_nodes, const int* node_types,
                                     const int* num_neigh, const int* neigh_indices, const int* neigh_types,
                                     const double* xyz, const double* r);

/* Largest displacement (A) measured by the last evaluation from positions
 * (sxl_compute_prepared_positions*): the same minimum-image displacement as
 * sxl_max_displacement, formed in that pass.  A caller may evaluate first
 * and rebuild and evaluate again when it breaks its skin rule, which saves
 * the separate check.  Invalid argument when the last evaluation was not
 * from positions or the graph changed since. */
int sxl_last_max_displacement(const sxl_evaluator* evaluator, double* out);

/* Largest minimum-image displacement of positions from the build's
 * fractional positions expressed in the current cell (the non-affine motion
 * of the skin-reuse rule, calculator.py:2851-2898). */
int sxl_max_displacement(sxl_evaluator* evaluator, uint64_t generation, const double* positions,
                         int positions_on_device, double* out);

/* LAMMPS pair_style symmetrix/mace on one rank: replaces
 * PairSymmetrixMACE::compute_no_domain_decomposition
 * (pair_symmetrix/pair_symmetrix_mace.cpp:309-441).  The arguments are the
 * pair style's own data: a full neighbour list (inum, ilist, numneigh and
 * firstneigh indexed by atom, entries masked with NEIGHMASK 0x1FFFFFFF) over
 * nall local + ghost atoms with coordinates x [nall][3] and 1-based types;
 * local_of[j] = atom->map(atom->tag[j]) maps every atom to its local atom;
 * mace_types [ntypes] is the pair_coeff map from LAMMPS type to model element.
 * Pairs with r < r_cut become edges i <- local_of[j]; f [nall][3] receives
 * f_i -= f_ij, f_local(j) += f_ij; energy (eng_vdwl) and virial [6] (xx yy zz
 * xy xz yz of sum xyz (x) f) are accumulated; eatom [nall] is set for local
 * atoms.  energy, eatom and virial may be null.  Invalid argument when a
 * neighbour maps to an atom outside ilist or a type is not mapped. */
int sxl_pair_compute(sxl_evaluator* evaluator, int inum, const int* ilist, const int* numneigh,
                     const int* const* firstneigh, int nall, const double* x, const int* type, const int* local_of,
                     int ntypes, const int* mace_types, double* f, double* energy, double* eatom, double* virial);

/* The same on the device arrays of a LAMMPS KOKKOS pair style (GPU build):
 * replaces PairSymmetrixMACEKokkos::compute_no_domain_decomposition
 * (pair_symmetrix/pair_symmetrix_mace_kokkos.cpp:1010-1260), which runs on
 * atomKK->k_x, k_list->d_ilist / d_numneigh / d_neighbors and k_f.  Every
 * array is in device memory except mace_types [ntypes] (host) and the
 * accumulators energy and virial [6] (host, may be null): ilist [inum],
 * numneigh [nall], neighbors with neighbour slot jj of atom i at
 * neighbors[i * neighbor_stride_atom + jj * neighbor_stride_slot] (masked with
 * NEIGHMASK; a Kokkos LayoutRight view has strides (maxneighs, 1), LayoutLeft
 * (1, rows)), x [nall][3], type [nall], local_of [nall], f [nall][3]
 * (accumulated) and eatom [nall] (set for local atoms, may be null).  The
 * list is filtered and mapped on the device and the graph prepared there;
 * only the per-atom neighbour counts come to the host.  Forces are the
 * evaluator's deterministic reduction of the directed forces (no atomics),
 * so the results equal sxl_pair_compute's on the same list bit for bit.  The
 * work runs on the evaluator's stream and has completed on return. */
int sxl_pair_compute_device(sxl_evaluator* evaluator, int inum, const int* d_ilist, const int* d_numneigh,
                            const int* d_neighbors, int64_t neighbor_stride_atom, int64_t neighbor_stride_slot,
                            int nall, const double* d_x, const int* d_type, const int* d_local_of, int ntypes,
                            const int* mace_types, double* d_f, double* energy, double* d_eatom, double* virial);

/* The KOKKOS pair style's prepared execution (the reference's path when the
 * model runs prepared graphs: pair_symmetrix/pair_symmetrix_mace_kokkos.cpp:
 * 1043-1160, its rebuild_topology condition and the stable edge set).
 * Arrays and accumulators as for sxl_pair_compute_device, except that every
 * listed pair becomes an edge: one at r >= r_cut is scaled to length r_cut
 * and contributes nothing.  With neighbor_ago = 0 (LAMMPS neighbor->ago: the
 * list was rebuilt this step), on the first call, when inum or nall changed
 * or when the evaluator prepared another graph in between, the graph is
 * rebuilt from the list; otherwise the list must be the previous call's and
 * only the edge vectors are formed from x before the prepared graph is
 * evaluated again (no host round trip for the topology).  An entry whose
 * neighbour count differs from the prepared graph's is an invalid-argument
 * error.  *rebuilt (may be null) is set to 1 when the graph was rebuilt.
 * Results match sxl_pair_compute_device's on the same list and positions to
 * FP32 rounding: the scaled pairs are inactive in every kernel but change
 * which of a receiver's edges share a kernel tile, so sums run in another
 * order; models with density-normalised layers also take every graph
 * neighbour into their density sums, as the reference's prepared execution
 * does.  Results are run-to-run identical. */
int sxl_pair_compute_device_prepared(sxl_evaluator* evaluator, int neighbor_ago, int inum, const int* d_ilist,
                                     const int* d_numneigh, const int* d_neighbors, int64_t neighbor_stride_atom,
                                     int64_t neighbor_stride_slot, int nall, const double* d_x, const int* d_type,
                                     const int* d_local_of, int ntypes, const int* mace_types, double* d_f,
                                     double* energy, double* d_eatom, double* virial, int* rebuilt);

/* Velocity-Verlet NVE molecular dynamics with positions, velocities and
 * forces resident on the device: the update of LAMMPS `fix nve` that the
 * reference's capacity runs apply with pair_style symmetrix/mace
 * (pair_symmetrix/pair_symmetrix_mace.cpp:309-441 supplies the forces).  Per
 * step: v += dt/2 F/m, x += dt v, forces at x, v += dt/2 F/m, with F/m in
 * A/fs^2 from eV/A and amu.  positions [N][3] (A) and velocities [N][3]
 * (A/fs) are read and overwritten with the final state; masses [N] in amu;
 * node_types are model element indices; dt in fs.  The periodic graph is
 * built on the device at r_cut + skin and rebuilt whenever an atom has moved
 * more than skin/2.  potential_energy and kinetic_energy (eV, steps + 1
 * values each, may be null) receive the energies after every step (index 0:
 * the start); step_seconds (steps values, may be null) the wall time of each
 * step with its work completed; rebuilds (may be null) the number of rebuilds
 * after the first build.  Leaves the last step's graph prepared. */
int sxl_md_nve(sxl_evaluator* evaluator, int num_atoms, const int* node_types, const double* masses,
               double* positions, double* velocities, const double* cell, const double* inverse_cell, double skin,
               double dt, int steps, double* potential_energy, double* kinetic_energy, double* step_seconds,
               int* rebuilds);
/* Progress of sxl_md_nve, the thermo output of LAMMPS `fix nve` runs (no
 * single reference counterpart): called on the calling thread after every
 * step (1-based) with the step's potential and kinetic energy (eV; NaN when
 * the run does not compute them) and its wall time (s); a nonzero return
 * ends the run after that step.  NULL removes it. */
typedef int (*sxl_md_progress_fn)(int step, double potential_energy, double kinetic_energy, double seconds,
                                  void* user);
int sxl_set_md_progress(sxl_evaluator* evaluator, sxl_md_progress_fn callback, void* user);

/* node_energies property, N doubles (mace_kokkos.cpp:2086-2093). */
int sxl_node_energies(const sxl_evaluator* evaluator, double* out, int num_nodes);
/* node_forces property, directed edge forces [E][3] (mace_kokkos.cpp:2094-2101). */
int sxl_node_forces(const sxl_evaluator* evaluator, double* out, int64_t num_edges);
/* _reduce_atom_forces: [N][3] (mace_kokkos.cpp:2103-2133). */
int sxl_reduce_atom_forces(sxl_evaluator* evaluator, uint64_t generation, double* out);
/* _reduce_stress(volume): 3x3 row-major (mace_kokkos.cpp:2134-2154). */
int sxl_reduce_stress(sxl_evaluator* evaluator, uint64_t generation, double volume, double* out9);
/* Sum of node energies in double (calculator.py:3831-3834). */
int sxl_total_energy(sxl_evaluator* evaluator, uint64_t generation, double* out);

/* Device pointers of the last evaluation's results, valid until the next
 * call: atom forces [N][3] and totals [10] = (energy, stress row-major); the
 * totals hold the stress of the last sxl_reduce_stress volume. */
int sxl_device_results(const sxl_evaluator* evaluator, const double** atom_forces, const double** totals);

int sxl_graph_size(const sxl_evaluator* evaluator, int* num_nodes, int64_t* num_edges, uint64_t* generation);

/* Model-free periodic neighbour graph on the device.  Replaces
 * build_periodic_neighbor_graph_kokkos(positions, cell, inverse_cell, cutoff)
 * (libsymmetrix/source/neighbor_graph_kokkos.cpp:38-405), whose Python
 * binding is _kokkos_periodic_neighbor_graph.  Build, then copy the arrays
 * (sized by num_edges) with sxl_neighbor_graph_copy, then free. */
typedef struct sxl_graph sxl_graph;
int sxl_neighbor_graph_build(const double* positions, int num_nodes, const double* cell,
                             const double* inverse_cell, double cutoff, sxl_graph** out, int64_t* num_edges);
int sxl_neighbor_graph_copy(const sxl_graph* graph, int* num_neigh, int* receiver_offsets, int* sources,
                            int* shifts, double* fractional_xyz);
void sxl_neighbor_graph_free(sxl_graph* graph);

/* No counterpart in the reference.  An allocation-free variant of
 * sxl_neighbor_graph_build for callers that cannot allocate device memory
 * (tight serving loops, harnesses that forbid hipMalloc): the same kernels and the same, bit-identical, edge list, with
 * the positions [N][3] and every output in the caller's device memory --
 * receiver_offsets [N+1], sources [edge_capacity], shifts and
 * fractional_xyz [edge_capacity][3] -- and the build's intermediate arrays
 * in one fixed device array of the library (SXL_NOALLOC_SCRATCH_BYTES per
 * GPU, held until the process ends).  No hipMalloc, hipFree or allocating
 * library call is made.  cell and inverse_cell are host arrays.  At most
 * SXL_NOALLOC_MAX_ATOMS atoms and SXL_NOALLOC_MAX_BINS cell bins (cell face
 * height / cutoff per axis, multiplied); more is a length error.  *num_edges
 * receives the edge count; when it exceeds edge_capacity the call returns a
 * length error and writes no output array (call again with larger arrays).
 * The work runs on `stream` (a hipStream_t; NULL: the default stream) and has
 * completed when the call returns: the call reads the edge count back to the
 * host and waits on the stream, so it cannot be recorded into a HIP graph
 * (stream capture).  All calls on one GPU share the library's
 * array: calls that overlap on one GPU (other threads, other streams) race. */
#define SXL_NOALLOC_MAX_ATOMS 131072
#define SXL_NOALLOC_MAX_BINS 262144
#define SXL_NOALLOC_SCRATCH_BYTES 18353408 /* about 17.5 MiB */
int sxl_neighbor_graph_build_noalloc(const double* d_positions, int num_nodes, const double* cell,
                                     const double* inverse_cell, double cutoff, int64_t edge_capacity,
                                     int* d_receiver_offsets, int* d_sources, int* d_shifts, double* d_fractional_xyz,
                                     int64_t* num_edges, void* stream);
/* Limits of sxl_neighbor_graph_build_noalloc (atoms and bins, may be NULL);
 * returns the bytes of its device array (SXL_NOALLOC_SCRATCH_BYTES). */
int64_t sxl_neighbor_graph_noalloc_limits(int* max_atoms, int* max_bins);
int sxl_stats(const sxl_evaluator* evaluator, sxl_stats_t* out);
/* Stage profiling: with enable != 0 every evaluation records HIP events
 * around each stage on the evaluator's stream (counters reset).  The
 * accumulated device time (ms) and count of each stage are read with
 * sxl_stage_times (arrays of sxl_num_stages() entries); sxl_stage_name gives
 * the stage names (kernel families).  Counterpart of the reference's
 * factorized_last_evaluation_ms timing fields (mace_kokkos.hpp:1425-1455). */
int sxl_set_profiling(sxl_evaluator* evaluator, int enable);
/* Profile only the stages whose bit is set in mask (bit i = stage i; 0 turns
 * profiling off): two events per profiled stage and evaluation. */
int sxl_set_profiling_stages(sxl_evaluator* evaluator, uint32_t mask);
/* HIP graph replay of evaluations from positions (sxl_compute_prepared_positions
 * and its device form) under the untiled plan: with enable != 0 the kernels of
 * such an evaluation, from the positions copy to the energy and stress
 * reduction, are captured into a HIP graph on the first call for a graph
 * generation, positions array and cell, and later calls replay it with one
 * launch (the result copies and the wait stay outside the graph); a new
 * graph, cell, reference geometry or positions array recaptures, profiling
 * evaluates eagerly.  For small graphs, whose evaluation is bound by the
 * host's kernel launches.  No reference counterpart (the reference runs
 * Kokkos kernels eagerly); off by default. */
int sxl_set_graph_replay(sxl_evaluator* evaluator, int enable);
int sxl_graph_replay(const sxl_evaluator* evaluator, int* enabled);
int sxl_num_stages(void);
const char* sxl_stage_name(int stage);
int sxl_stage_times(const sxl_evaluator* evaluator, double* ms, int* counts);

/* Execution-plan request (_set_execution_plan_request,
 * mace_kokkos.cpp:266-269): algorithm "direct"; profile "capacity" (receiver
 * tiles when the untiled estimate exceeds the memory budget and fixed
 * workspace is allowed) or "speed" (untiled); debug_plan NULL/"" or
 * "mh0-direct-speed" / "mh0-dual-layer-tiled-v1" to pin a plan.  Invalidates
 * the prepared graph. */
int sxl_set_execution_plan_request(sxl_evaluator* evaluator, const char* algorithm, const char* profile,
                                   const char* debug_plan);

/* selected_head and available_heads of the loaded model
 * (mace_kokkos.cpp:1904-1905; head selection prediction_heads.hpp:10-89) as
 * a JSON object {"selected_head": ..., "available_heads": [...]}; buffer,
 * capacity and length as for sxl_execution_plan_json. */
int sxl_model_heads_json(const sxl_evaluator* evaluator, char* buffer, int64_t capacity, int64_t* length);

/* execution_plan_report property (mace_kokkos.cpp:271-297) as a JSON object
 * with the reference's fields: requested_algorithm, requested_profile,
 * selection_source, state, selected_id, selection_reason, available_bytes,
 * reserve_bytes, boundary_attempt, candidates [{id, qualified,
 * estimated_bytes, reason}].  *length receives the text length; with a
 * non-null buffer the text and a NUL are written (length error when capacity
 * is not larger than the length). */
int sxl_execution_plan_json(const sxl_evaluator* evaluator, char* buffer, int64_t capacity, int64_t* length);

/* Device memory by role and the plan's capacities of the prepared graph, as
 * a JSON object of integers: graph_generation, num_nodes, num_edges, tiled,
 * tile_receivers, num_tiles, max_tile_edges, tile_runs, run_bytes,
 * graph_bytes, geometry_bytes, node_work_bytes, edge_work_bytes, phi1_bytes,
 * message_bytes, readout_bytes, feature_bytes, reduction_bytes, table_bytes,
 * device_free_bytes, device_total_bytes, a0_unfolded, r1_forward_slices,
 * r1_reverse_slices, a0_forward_slices, edge_tile (edges per tile of the
 * reverse edge kernels' tile launches, 0 without).  The source of the
 * reference's workspace and policy
 * properties (phi1_workspace_bytes, readout_workspace_bytes,
 * dual_layer_workspace_*, execution_planned_*, low_memory_*;
 * symmetrix/source/cpp/mace_kokkos.cpp:517-630,
 * libsymmetrix/source/mace_kokkos_runtime.cpp:2366-2511, 4093-4336).
 * Buffer, capacity and length as for sxl_execution_plan_json. */
int sxl_workspace_json(const sxl_evaluator* evaluator, char* buffer, int64_t capacity, int64_t* length);

/* Tiled ("fixed workspace") execution for capacity runs: receivers are
 * processed in tiles with one reused work arena; graph-wide state is H1, its
 * adjoint and two per-node scalar blocks.  With allow != 0 the plan of the
 * next prepared graph is tiled when the receiver limit (if set) is below the
 * node count, or when the untiled work arrays would not fit the free device
 * memory (tiles of 32768 receivers).  Both setters invalidate the prepared
 * graph: prepare again afterwards.  Replace MACEKokkos::set_allow_fixed_workspace
 * (libsymmetrix/source/mace_kokkos_runtime.cpp:3992-4000; Python
 * _set_allow_fixed_workspace, symmetrix/source/cpp/mace_kokkos.cpp:444-447)
 * and set_dual_layer_workspace_receiver_limit_for_testing
 * (mace_kokkos_runtime.cpp:2771-2781; Python binding mace_kokkos.cpp:439-441);
 * a limit <= 0 is rejected like the reference's. */
int sxl_set_allow_fixed_workspace(sxl_evaluator* evaluator, int allow);
int sxl_allow_fixed_workspace(const sxl_evaluator* evaluator, int* allow);
int sxl_set_workspace_receiver_limit(sxl_evaluator* evaluator, int receivers);

/* Waits for all device work of the evaluator. */
int sxl_synchronize(const sxl_evaluator* evaluator);

#ifdef __cplusplus
}
#endif

#endif /* SYMMETRIX_AMD_H */
