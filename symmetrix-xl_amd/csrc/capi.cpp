// C ABI of the evaluator (include/symmetrix_amd.h): exception-free wrappers.
#include "../../include/symmetrix_amd.h"

#include <algorithm>
#include <cmath>
#include <memory>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "evaluator.hpp"
#include "pair.hpp"

struct sxl_evaluator {
    sxl::Evaluator impl;
    sxl::PairDriver pair;
    sxl_evaluator(const char* path, const char* head) : impl(path, head ? head : "") {}
};

struct sxl_graph {
    sxl::PeriodicGraph graph;
};

namespace {

thread_local std::string g_error;

template <class F>
int guarded(F&& f)
{
    try {
        f();
        g_error.clear();
        return SXL_OK;
    } catch (const std::bad_alloc& e) {
        g_error = e.what();
        return SXL_ALLOCATION_ERROR;
    } catch (const std::out_of_range& e) {
        g_error = e.what();
        return SXL_OUT_OF_RANGE;
    } catch (const std::length_error& e) {
        g_error = e.what();
        return SXL_LENGTH_ERROR;
    } catch (const std::invalid_argument& e) {
        g_error = e.what();
        return SXL_INVALID_ARGUMENT;
    } catch (const std::logic_error& e) {
        g_error = e.what();
        return SXL_LOGIC_ERROR;
    } catch (const std::exception& e) {
        g_error = e.what();
        return SXL_RUNTIME_ERROR;
    } catch (...) {
        g_error = "unknown error";
        return SXL_RUNTIME_ERROR;
    }
}

int null_handle()
{
    g_error = "null evaluator handle or output pointer";
    return SXL_INVALID_ARGUMENT;
}

// Runtime lifecycle (reference libsymmetrix/source/tools_kokkos.cpp:44-99):
// evaluators are counted while alive; finalization is refused while any is
// alive and is final -- no evaluator can be constructed afterwards.
std::mutex g_runtime_mutex;
bool g_runtime_initialized = false;
bool g_runtime_finalized = false;
std::int64_t g_live_evaluators = 0;

void initialize_runtime_locked()
{
    if (g_runtime_finalized) throw std::runtime_error("Cannot initialize the HIP runtime after finalization.");
    if (g_runtime_initialized) return;
    const hipError_t err = hipInit(0);
    int devices = 0;
    if (err != hipSuccess || hipGetDeviceCount(&devices) != hipSuccess || devices <= 0) {
        (void)hipGetLastError();
        throw std::runtime_error("HIP runtime initialization found no usable device.");
    }
    g_runtime_initialized = true;
}

}  // namespace

extern "C" {

const char* sxl_last_error(void) { return g_error.c_str(); }

int sxl_create(const char* model_path, const char* head, sxl_evaluator** out)
{
    if (!model_path || !out) return null_handle();
    *out = nullptr;
    return guarded([&] {
        {
            const std::scoped_lock lock(g_runtime_mutex);
            if (g_runtime_finalized)
                throw std::runtime_error("Cannot construct a Symmetrix evaluator after Kokkos finalization.");
        }
        auto ev = std::make_unique<sxl_evaluator>(model_path, head);
        const std::scoped_lock lock(g_runtime_mutex);
        // a finalization that ran while this evaluator was being built wins
        if (g_runtime_finalized)
            throw std::runtime_error("Cannot construct a Symmetrix evaluator after Kokkos finalization.");
        g_runtime_initialized = true;
        g_live_evaluators += 1;
        *out = ev.release();
    });
}

void sxl_destroy(sxl_evaluator* evaluator)
{
    if (!evaluator) return;
    delete evaluator;
    const std::scoped_lock lock(g_runtime_mutex);
    g_live_evaluators -= 1;
}

int sxl_runtime_initialize(void)
{
    return guarded([] {
        const std::scoped_lock lock(g_runtime_mutex);
        initialize_runtime_locked();
    });
}

int sxl_runtime_finalize(void)
{
    return guarded([] {
        const std::scoped_lock lock(g_runtime_mutex);
        if (g_live_evaluators != 0)
            throw std::runtime_error("Cannot finalize Kokkos while " + std::to_string(g_live_evaluators) +
                                     " Symmetrix evaluator object(s) are alive.");
        g_runtime_initialized = false;
        g_runtime_finalized = true;
    });
}

int sxl_runtime_is_initialized(void)
{
    const std::scoped_lock lock(g_runtime_mutex);
    return g_runtime_initialized ? 1 : 0;
}

int64_t sxl_live_evaluator_count(void)
{
    const std::scoped_lock lock(g_runtime_mutex);
    return g_live_evaluators;
}

const char* sxl_default_execution_space(void) { return "HIP"; }

int sxl_model_info(const sxl_evaluator* ev, sxl_model_info_t* out)
{
    if (!ev || !out) return null_handle();
    return guarded([&] {
        const sxl::HostModel& m = ev->impl.model();
        out->num_elements = m.num_elements;
        out->num_channels = m.channels;
        out->l_max = m.l_max;
        out->L_max = m.L_max;
        out->num_paths = m.num_paths();
        out->spline_points = m.spline_points;
        out->r_cut = m.r_cut;
    });
}

int sxl_atomic_numbers(const sxl_evaluator* ev, int* out)
{
    if (!ev || !out) return null_handle();
    return guarded([&] {
        const auto& v = ev->impl.model().atomic_numbers;
        for (std::size_t i = 0; i < v.size(); ++i) out[i] = v[i];
    });
}

int sxl_atomic_energies(const sxl_evaluator* ev, double* out)
{
    if (!ev || !out) return null_handle();
    return guarded([&] {
        const auto& v = ev->impl.model().atomic_energies;
        for (std::size_t i = 0; i < v.size(); ++i) out[i] = v[i];
    });
}

int sxl_prepare_graph(sxl_evaluator* ev, int num_nodes, const int* node_types, const int* num_neigh,
                      const int* neigh_indices, const int* neigh_types, uint64_t* generation)
{
    if (!ev || !generation || (num_nodes > 0 && (!node_types || !num_neigh))) return null_handle();
    return guarded([&] {
        *generation = ev->impl.prepare_graph(num_nodes, node_types, num_neigh, neigh_indices, neigh_types);
    });
}

int sxl_prepare_graph_device(sxl_evaluator* ev, int num_nodes, const int* d_node_types, const int* d_num_neigh,
                             const int* d_neigh_indices, const int* d_neigh_types, uint64_t* generation)
{
    if (!ev || !generation || (num_nodes > 0 && (!d_node_types || !d_num_neigh))) return null_handle();
    return guarded([&] {
        *generation =
            ev->impl.prepare_graph_device(num_nodes, d_node_types, d_num_neigh, d_neigh_indices, d_neigh_types);
    });
}

static int prepare_periodic(sxl_evaluator* ev, int num_nodes, const int* node_types, const double* positions,
                            bool device, const double* cell, const double* inverse_cell, double cutoff,
                            uint64_t* generation, int64_t* num_edges)
{
    if (!ev || !generation || !cell || !inverse_cell || (num_nodes > 0 && (!node_types || !positions)))
        return null_handle();
    return guarded([&] {
        *generation = ev->impl.prepare_periodic_graph(num_nodes, node_types, positions, device, cell, inverse_cell,
                                                      cutoff);
        if (num_edges) *num_edges = ev->impl.num_edges();
    });
}

int sxl_prepare_periodic_graph(sxl_evaluator* ev, int num_nodes, const int* node_types, const double* positions,
                               const double* cell, const double* inverse_cell, double cutoff, uint64_t* generation,
                               int64_t* num_edges)
{
    return prepare_periodic(ev, num_nodes, node_types, positions, false, cell, inverse_cell, cutoff, generation,
                            num_edges);
}

int sxl_prepare_periodic_graph_device(sxl_evaluator* ev, int num_nodes, const int* node_types,
                                      const double* d_positions, const double* cell, const double* inverse_cell,
                                      double cutoff, uint64_t* generation, int64_t* num_edges)
{
    return prepare_periodic(ev, num_nodes, node_types, d_positions, true, cell, inverse_cell, cutoff, generation,
                            num_edges);
}

int sxl_graph_arrays(sxl_evaluator* ev, uint64_t generation, int* num_neigh, int* receiver_offsets, int* sources,
                     int* shifts, double* fractional_xyz)
{
    if (!ev) return null_handle();
    return guarded(
        [&] { ev->impl.graph_arrays(generation, num_neigh, receiver_offsets, sources, shifts, fractional_xyz); });
}

int sxl_update_cell(sxl_evaluator* ev, uint64_t generation, const double* cell, const double* inverse_cell)
{
    if (!ev || !cell || !inverse_cell) return null_handle();
    return guarded([&] { ev->impl.update_cell(generation, cell, inverse_cell); });
}

int sxl_validate_graph_cardinality(const sxl_evaluator* ev, int64_t num_receivers, int64_t num_feature_nodes,
                                   int64_t num_edges)
{
    if (!ev) return null_handle();
    return guarded([&] {
        if (num_receivers < 0 || num_feature_nodes < 0 || num_edges < 0)
            throw std::invalid_argument("MACE graph cardinalities must be non-negative.");
        ev->impl.validate_graph_cardinality(static_cast<uint64_t>(num_receivers),
                                            static_cast<uint64_t>(num_feature_nodes),
                                            static_cast<uint64_t>(num_edges));
    });
}

int sxl_prepare_geometry(sxl_evaluator* ev, uint64_t generation, const double* reference_positions,
                         int64_t num_positions, const double* reference_xyz, int64_t num_xyz, const double* cell,
                         const double* inverse_cell, const int* pbc)
{
    if (!ev || !cell || !inverse_cell || !pbc || num_positions < 0 || num_xyz < 0 ||
        (num_positions > 0 && !reference_positions) || (num_xyz > 0 && !reference_xyz))
        return null_handle();
    return guarded([&] {
        ev->impl.prepare_geometry(generation, reference_positions, static_cast<std::size_t>(num_positions),
                                  reference_xyz, static_cast<std::size_t>(num_xyz), cell, inverse_cell, pbc, false);
    });
}

int sxl_prepare_fractional_geometry(sxl_evaluator* ev, uint64_t generation, const double* fractional_positions,
                                    int64_t num_positions, const double* fractional_xyz, int64_t num_xyz,
                                    const double* cell, const double* inverse_cell, const int* pbc)
{
    if (!ev || !cell || !inverse_cell || !pbc || num_positions < 0 || num_xyz < 0 ||
        (num_positions > 0 && !fractional_positions) || (num_xyz > 0 && !fractional_xyz))
        return null_handle();
    return guarded([&] {
        ev->impl.prepare_geometry(generation, fractional_positions, static_cast<std::size_t>(num_positions),
                                  fractional_xyz, static_cast<std::size_t>(num_xyz), cell, inverse_cell, pbc, true);
    });
}

int sxl_prepare_shift_geometry(sxl_evaluator* ev, uint64_t generation, const double* reference_positions,
                               int64_t num_positions, const int* shifts, int64_t num_shifts, const double* cell,
                               const double* inverse_cell, const int* pbc)
{
    if (!ev || !cell || !inverse_cell || !pbc || num_positions < 0 || num_shifts < 0 ||
        (num_positions > 0 && !reference_positions) || (num_shifts > 0 && !shifts))
        return null_handle();
    return guarded([&] {
        ev->impl.prepare_shift_geometry(generation, reference_positions, static_cast<std::size_t>(num_positions),
                                        shifts, static_cast<std::size_t>(num_shifts), cell, inverse_cell, pbc);
    });
}

int sxl_compute_prepared_positions(sxl_evaluator* ev, uint64_t generation, const double* positions)
{
    if (!ev || (!positions && ev->impl.num_nodes() > 0)) return null_handle();
    return guarded([&] { ev->impl.compute_positions(generation, positions, false); });
}

int sxl_compute_prepared_positions_device(sxl_evaluator* ev, uint64_t generation, const double* d_positions)
{
    if (!ev || (!d_positions && ev->impl.num_nodes() > 0)) return null_handle();
    return guarded([&] { ev->impl.compute_positions(generation, d_positions, true); });
}

int sxl_compute_prepared(sxl_evaluator* ev, uint64_t generation, const double* xyz, const double* r)
{
    if (!ev || ((!xyz || !r) && ev->impl.num_edges() > 0)) return null_handle();
    return guarded([&] { ev->impl.compute_xyz(generation, xyz, r, false); });
}

int sxl_compute_prepared_device(sxl_evaluator* ev, uint64_t generation, const double* d_xyz, const double* d_r)
{
    if (!ev || ((!d_xyz || !d_r) && ev->impl.num_edges() > 0)) return null_handle();
    return guarded([&] { ev->impl.compute_xyz(generation, d_xyz, d_r, true); });
}

int sxl_compute_node_energies_forces(sxl_evaluator* ev, int num_nodes, const int* node_types, const int* num_neigh,
                                     const int* neigh_indices, const int* neigh_types, const double* xyz,
                                     const double* r)
{
    if (!ev) return null_handle();
    return guarded([&] {
        const uint64_t g = ev->impl.prepare_graph(num_nodes, node_types, num_neigh, neigh_indices, neigh_types);
        ev->impl.compute_xyz(g, xyz, r, false);
    });
}

int sxl_max_displacement(sxl_evaluator* ev, uint64_t generation, const double* positions, int on_device,
                         double* out)
{
    if (!ev || !out) return null_handle();
    return guarded([&] { *out = ev->impl.max_displacement(generation, positions, on_device != 0); });
}

int sxl_pair_compute(sxl_evaluator* ev, int inum, const int* ilist, const int* numneigh,
                     const int* const* firstneigh, int nall, const double* x, const int* type, const int* local_of,
                     int ntypes, const int* mace_types, double* f, double* energy, double* eatom, double* virial)
{
    if (!ev || !f) return null_handle();
    return guarded([&] {
        sxl::PairInput in;
        in.inum = inum;
        in.ilist = ilist;
        in.numneigh = numneigh;
        in.firstneigh = firstneigh;
        in.nall = nall;
        in.x = x;
        in.type = type;
        in.local_of = local_of;
        in.ntypes = ntypes;
        in.mace_types = mace_types;
        sxl::PairOutput out;
        out.f = f;
        out.energy = energy;
        out.eatom = eatom;
        out.virial = virial;
        ev->pair.compute(ev->impl, in, out);
    });
}

int sxl_pair_compute_device(sxl_evaluator* ev, int inum, const int* d_ilist, const int* d_numneigh,
                            const int* d_neighbors, int64_t neighbor_stride_atom, int64_t neighbor_stride_slot,
                            int nall, const double* d_x, const int* d_type, const int* d_local_of, int ntypes,
                            const int* mace_types, double* d_f, double* energy, double* d_eatom, double* virial)
{
    if (!ev || !d_f) return null_handle();
    return guarded([&] {
        sxl::PairDeviceInput in;
        in.inum = inum;
        in.ilist = d_ilist;
        in.numneigh = d_numneigh;
        in.neighbors = d_neighbors;
        in.stride_atom = neighbor_stride_atom;
        in.stride_slot = neighbor_stride_slot;
        in.nall = nall;
        in.x = d_x;
        in.type = d_type;
        in.local_of = d_local_of;
        in.ntypes = ntypes;
        in.mace_types = mace_types;
        sxl::PairOutput out;
        out.f = d_f;
        out.energy = energy;
        out.eatom = d_eatom;
        out.virial = virial;
        ev->pair.compute_device(ev->impl, in, out);
    });
}

int sxl_pair_compute_device_prepared(sxl_evaluator* ev, int neighbor_ago, int inum, const int* d_ilist,
                                     const int* d_numneigh, const int* d_neighbors, int64_t neighbor_stride_atom,
                                     int64_t neighbor_stride_slot, int nall, const double* d_x, const int* d_type,
                                     const int* d_local_of, int ntypes, const int* mace_types, double* d_f,
                                     double* energy, double* d_eatom, double* virial, int* rebuilt)
{
    if (!ev || !d_f) return null_handle();
    return guarded([&] {
        sxl::PairDeviceInput in;
        in.inum = inum;
        in.ilist = d_ilist;
        in.numneigh = d_numneigh;
        in.neighbors = d_neighbors;
        in.stride_atom = neighbor_stride_atom;
        in.stride_slot = neighbor_stride_slot;
        in.nall = nall;
        in.x = d_x;
        in.type = d_type;
        in.local_of = d_local_of;
        in.ntypes = ntypes;
        in.mace_types = mace_types;
        sxl::PairOutput out;
        out.f = d_f;
        out.energy = energy;
        out.eatom = d_eatom;
        out.virial = virial;
        bool r = false;
        ev->pair.compute_device_prepared(ev->impl, neighbor_ago, in, out, &r);
        if (rebuilt) *rebuilt = r ? 1 : 0;
    });
}

int sxl_md_nve(sxl_evaluator* ev, int num_atoms, const int* node_types, const double* masses, double* positions,
               double* velocities, const double* cell, const double* inverse_cell, double skin, double dt, int steps,
               double* potential_energy, double* kinetic_energy, double* step_seconds, int* rebuilds)
{
    if (!ev || !node_types || !masses || !positions || !velocities || !cell || !inverse_cell) return null_handle();
    return guarded([&] {
        const int n = ev->impl.md_nve(num_atoms, node_types, masses, positions, velocities, cell, inverse_cell, skin,
                                      dt, steps, potential_energy, kinetic_energy, step_seconds);
        if (rebuilds) *rebuilds = n;
    });
}

int sxl_set_md_progress(sxl_evaluator* ev, sxl_md_progress_fn callback, void* user)
{
    if (!ev) return null_handle();
    return guarded([&] { ev->impl.set_md_progress(callback, user); });
}

int sxl_node_energies(const sxl_evaluator* ev, double* out, int num_nodes)
{
    if (!ev || (!out && num_nodes > 0)) return null_handle();
    return guarded([&] {
        if (num_nodes != ev->impl.num_nodes()) throw std::invalid_argument("node energy extent mismatch");
        ev->impl.node_energies(out);
    });
}

int sxl_node_forces(const sxl_evaluator* ev, double* out, int64_t num_edges)
{
    if (!ev || (!out && num_edges > 0)) return null_handle();
    return guarded([&] {
        if (num_edges != ev->impl.num_edges()) throw std::invalid_argument("directed force extent mismatch");
        ev->impl.node_forces(out);
    });
}

int sxl_reduce_atom_forces(sxl_evaluator* ev, uint64_t generation, double* out)
{
    if (!ev || (!out && ev->impl.num_nodes() > 0)) return null_handle();
    return guarded([&] { ev->impl.atom_forces(generation, out); });
}

int sxl_reduce_stress(sxl_evaluator* ev, uint64_t generation, double volume, double* out9)
{
    if (!ev || !out9) return null_handle();
    return guarded([&] { ev->impl.stress(generation, volume, out9); });
}

int sxl_total_energy(sxl_evaluator* ev, uint64_t generation, double* out)
{
    if (!ev || !out) return null_handle();
    return guarded([&] { *out = ev->impl.total_energy(generation); });
}

int sxl_device_results(const sxl_evaluator* ev, const double** atom_forces, const double** totals)
{
    if (!ev) return null_handle();
    return guarded([&] {
        if (atom_forces) *atom_forces = ev->impl.device_atom_forces();
        if (totals) *totals = ev->impl.device_totals();
    });
}

int sxl_graph_size(const sxl_evaluator* ev, int* num_nodes, int64_t* num_edges, uint64_t* generation)
{
    if (!ev) return null_handle();
    return guarded([&] {
        if (num_nodes) *num_nodes = ev->impl.num_nodes();
        if (num_edges) *num_edges = ev->impl.num_edges();
        if (generation) *generation = ev->impl.generation();
    });
}

int sxl_stats(const sxl_evaluator* ev, sxl_stats_t* out)
{
    if (!ev || !out) return null_handle();
    return guarded([&] {
        const sxl::EvaluatorStats& s = ev->impl.stats();
        out->num_nodes = ev->impl.num_nodes();
        out->num_edges = ev->impl.num_edges();
        out->graph_builds = s.graph_builds;
        out->evaluations = s.evaluations;
        out->last_evaluation_ms = s.last_evaluation_ms;
        out->device_bytes = static_cast<int64_t>(sxl::device_bytes_in_use());
        out->tiled_evaluations = s.tiled_evaluations;
        out->tile_receivers = s.tile_receivers;
        out->num_tiles = s.num_tiles;
        out->last_graph_prepare_ms = s.last_graph_prepare_ms;
        out->preparation_fences = s.preparation_fences;
        out->evaluation_fences = s.evaluation_fences;
        out->last_evaluation_launches = s.last_evaluation_launches;
        out->last_evaluation_allocations = s.last_evaluation_allocations;
        out->last_evaluation_fences = s.last_evaluation_fences;
    });
}

int sxl_set_allow_fixed_workspace(sxl_evaluator* ev, int allow)
{
    if (!ev) return null_handle();
    return guarded([&] { ev->impl.set_allow_fixed_workspace(allow != 0); });
}

int sxl_allow_fixed_workspace(const sxl_evaluator* ev, int* allow)
{
    if (!ev || !allow) return null_handle();
    return guarded([&] { *allow = ev->impl.allow_fixed_workspace() ? 1 : 0; });
}

int sxl_set_execution_plan_request(sxl_evaluator* ev, const char* algorithm, const char* profile,
                                   const char* debug_plan)
{
    if (!ev || !algorithm || !profile) return null_handle();
    return guarded([&] { ev->impl.set_execution_plan_request(algorithm, profile, debug_plan ? debug_plan : ""); });
}

int sxl_model_heads_json(const sxl_evaluator* ev, char* buffer, int64_t capacity, int64_t* length)
{
    if (!ev || !length) return null_handle();
    return guarded([&] {
        const sxl::HostModel& m = ev->impl.model();
        auto quote = [](const std::string& v) {
            std::string out = "\"";
            for (char c : v) {
                if (c == '"' || c == '\\') out += '\\';
                out += c;
            }
            return out + "\"";
        };
        std::string text = "{\"selected_head\": " + quote(m.selected_head) + ", \"available_heads\": [";
        for (std::size_t i = 0; i < m.available_heads.size(); ++i)
            text += (i ? ", " : "") + quote(m.available_heads[i]);
        text += "]}";
        *length = static_cast<int64_t>(text.size());
        if (!buffer) return;
        if (capacity <= static_cast<int64_t>(text.size()))
            throw std::length_error("head buffer is smaller than the report");
        std::copy(text.begin(), text.end(), buffer);
        buffer[text.size()] = '\0';
    });
}

int sxl_execution_plan_json(const sxl_evaluator* ev, char* buffer, int64_t capacity, int64_t* length)
{
    if (!ev || !length) return null_handle();
    return guarded([&] {
        const std::string text = ev->impl.execution_plan_report().json();
        *length = static_cast<int64_t>(text.size());
        if (!buffer) return;
        if (capacity <= static_cast<int64_t>(text.size()))
            throw std::length_error("execution-plan buffer is smaller than the report");
        std::copy(text.begin(), text.end(), buffer);
        buffer[text.size()] = '\0';
    });
}

int sxl_workspace_json(const sxl_evaluator* ev, char* buffer, int64_t capacity, int64_t* length)
{
    if (!ev || !length) return null_handle();
    return guarded([&] {
        const std::string text = ev->impl.workspace_json();
        *length = static_cast<int64_t>(text.size());
        if (!buffer) return;
        if (capacity <= static_cast<int64_t>(text.size()))
            throw std::length_error("workspace buffer is smaller than the report");
        std::copy(text.begin(), text.end(), buffer);
        buffer[text.size()] = '\0';
    });
}

int sxl_set_workspace_receiver_limit(sxl_evaluator* ev, int receivers)
{
    if (!ev) return null_handle();
    return guarded([&] { ev->impl.set_workspace_receiver_limit(receivers); });
}

int sxl_neighbor_graph_build(const double* positions, int num_nodes, const double* cell, const double* inverse_cell,
                             double cutoff, sxl_graph** out, int64_t* num_edges)
{
    if (!out || !cell || !inverse_cell || (num_nodes > 0 && !positions)) return null_handle();
    *out = nullptr;
    return guarded([&] {
        sxl::validate_periodic_inputs(num_nodes, cell, inverse_cell, cutoff);
        for (long long i = 0; i < 3LL * num_nodes; ++i)
            if (!std::isfinite(positions[i])) throw std::invalid_argument("neighbor graph positions must be finite");
        hipStream_t stream = nullptr;
        if (hipStreamCreateWithFlags(&stream, hipStreamNonBlocking) != hipSuccess)
            throw std::runtime_error("stream creation failed");
        auto graph = std::make_unique<sxl_graph>();
        try {
            sxl::DeviceBuffer d_pos;
            d_pos.reserve(std::max(num_nodes, 1) * 3 * sizeof(double));
            if (num_nodes > 0 &&
                hipMemcpy(d_pos.as<double>(), positions, num_nodes * 3 * sizeof(double), hipMemcpyHostToDevice) !=
                    hipSuccess)
                throw std::runtime_error("position upload failed");
            sxl::build_periodic_graph(d_pos.as<double>(), num_nodes, cell, inverse_cell, cutoff, stream, graph->graph);
        } catch (...) {
            (void)hipStreamDestroy(stream);
            throw;
        }
        (void)hipStreamDestroy(stream);
        if (num_edges) *num_edges = graph->graph.num_edges;
        *out = graph.release();
    });
}

int sxl_neighbor_graph_copy(const sxl_graph* g, int* num_neigh, int* receiver_offsets, int* sources, int* shifts,
                            double* fractional_xyz)
{
    if (!g) return null_handle();
    return guarded([&] {
        const int N = g->graph.num_nodes;
        const long long E = g->graph.num_edges;
        std::vector<int> first(N + 1);
        auto copy = [](void* dst, const void* src, size_t bytes) {
            if (bytes && hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost) != hipSuccess)
                throw std::runtime_error("graph copy failed");
        };
        copy(first.data(), g->graph.first.as<int>(), (N + 1) * sizeof(int));
        if (receiver_offsets) std::copy(first.begin(), first.end(), receiver_offsets);
        if (num_neigh)
            for (int i = 0; i < N; ++i) num_neigh[i] = first[i + 1] - first[i];
        if (sources) copy(sources, g->graph.sources.as<int>(), E * sizeof(int));
        if (shifts) copy(shifts, g->graph.shifts.as<int>(), E * 3 * sizeof(int));
        if (fractional_xyz) copy(fractional_xyz, g->graph.fractional_xyz.as<double>(), E * 3 * sizeof(double));
    });
}

void sxl_neighbor_graph_free(sxl_graph* graph) { delete graph; }

int sxl_neighbor_graph_build_noalloc(const double* d_positions, int num_nodes, const double* cell,
                                     const double* inverse_cell, double cutoff, int64_t edge_capacity,
                                     int* d_receiver_offsets, int* d_sources, int* d_shifts, double* d_fractional_xyz,
                                     int64_t* num_edges, void* stream)
{
    if (!cell || !inverse_cell || !num_edges || !d_receiver_offsets || (num_nodes > 0 && !d_positions) ||
        (edge_capacity > 0 && (!d_sources || !d_shifts || !d_fractional_xyz)))
        return null_handle();
    *num_edges = 0;
    return guarded([&] {
        long long edges = 0;
        try {
            sxl::build_periodic_graph_noalloc(d_positions, num_nodes, cell, inverse_cell, cutoff, edge_capacity,
                                              d_receiver_offsets, d_sources, d_shifts, d_fractional_xyz, &edges,
                                              static_cast<hipStream_t>(stream));
        } catch (...) {
            *num_edges = edges;
            throw;
        }
        *num_edges = edges;
    });
}

int64_t sxl_neighbor_graph_noalloc_limits(int* max_atoms, int* max_bins)
{
    if (max_atoms) *max_atoms = sxl::kNoAllocMaxAtoms;
    if (max_bins) *max_bins = sxl::kNoAllocMaxBins;
    return static_cast<int64_t>(sxl::noalloc_scratch_bytes());
}

int sxl_set_profiling_stages(sxl_evaluator* ev, uint32_t mask)
{
    if (!ev) return null_handle();
    return guarded([&] { ev->impl.set_profiling_stages(mask); });
}

int sxl_last_max_displacement(const sxl_evaluator* ev, double* out)
{
    if (!ev || !out) return null_handle();
    return guarded([&] { *out = ev->impl.last_max_displacement(); });
}

int sxl_set_profiling(sxl_evaluator* ev, int enable)
{
    if (!ev) return null_handle();
    return guarded([&] { ev->impl.set_profiling(enable != 0); });
}

int sxl_set_graph_replay(sxl_evaluator* ev, int enable)
{
    if (!ev) return null_handle();
    return guarded([&] { ev->impl.set_graph_replay(enable != 0); });
}

int sxl_graph_replay(const sxl_evaluator* ev, int* enabled)
{
    if (!ev || !enabled) return null_handle();
    return guarded([&] { *enabled = ev->impl.graph_replay() ? 1 : 0; });
}

int sxl_num_stages(void) { return sxl::kNumStages; }

const char* sxl_stage_name(int stage) { return sxl::stage_name(stage); }

int sxl_stage_times(const sxl_evaluator* ev, double* ms, int* counts)
{
    if (!ev) return null_handle();
    return guarded([&] { ev->impl.stage_times(ms, counts); });
}

int sxl_synchronize(const sxl_evaluator* ev)
{
    if (!ev) return null_handle();
    return guarded([&] { ev->impl.synchronize(); });
}

}  // extern "C"
