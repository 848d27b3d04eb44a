/*
 * C++ facade of the MI355X MACE evaluator: the methods of the reference's
 * MACEKokkos<float> on the energy / force / stress path, with the same names,
 * argument order and meaning (libsymmetrix/source/mace_kokkos.hpp:91-97,
 * 339-460, 489-501, 654-710), over the C-ABI of symmetrix_amd.h.  Header
 * only, C++20 (std::span, as the reference).
 *
 * Differences a caller sees:
 *   - the class is symmetrix_amd::MACEKokkosFloat, FP32 only (the reference
 *     template is instantiated for float by the GPU builds);
 *   - spans are host arrays (the reference's *_device overloads take
 *     Kokkos::View; this build has no Kokkos);
 *   - node_energies / node_forces / atom_forces / stress_tensor are accessor
 *     calls returning host copies of the last evaluation's results (the
 *     reference exposes device views as members); they are fetched on first
 *     access after an evaluation;
 *   - errors are the reference's exception types (std::invalid_argument,
 *     std::out_of_range, std::length_error, std::runtime_error,
 *     std::logic_error) carrying the library's message; allocation failures
 *     are std::runtime_error with the message.
 * One object owns one evaluator (one HIP stream); it is not thread-safe, as
 * the reference's is not.
 */
#pragma once

#include <cstddef>
#include <cstdint>
#include <span>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "symmetrix_amd.h"

namespace symmetrix_amd {

namespace detail {

inline void check(int status)
{
    if (status == SXL_OK) return;
    const char* text = sxl_last_error();
    const std::string message = text ? text : "";
    switch (status) {
    case SXL_INVALID_ARGUMENT: throw std::invalid_argument(message);
    case SXL_OUT_OF_RANGE: throw std::out_of_range(message);
    case SXL_LENGTH_ERROR: throw std::length_error(message);
    case SXL_LOGIC_ERROR: throw std::logic_error(message);
    default: throw std::runtime_error(message);
    }
}

inline void require(bool condition, const char* message)
{
    if (!condition) throw std::invalid_argument(message);
}

// JSON text from a (buffer, capacity, length) query: sized by a first call.
template <class Query>
std::string json_text(Query query)
{
    std::int64_t length = 0;
    check(query(nullptr, 0, &length));
    std::string text(static_cast<std::size_t>(length), '\0');
    check(query(text.data(), length + 1, &length));
    return text;
}

// the quoted strings in text[begin, end) (the library escapes '"' and '\\'
// with a backslash)
inline std::vector<std::string> json_strings(const std::string& text, std::size_t begin, std::size_t end)
{
    std::vector<std::string> out;
    end = end < text.size() ? end : text.size();
    for (std::size_t i = begin; i < end; ++i) {
        if (text[i] != '"') continue;
        std::string value;
        for (++i; i < text.size() && text[i] != '"'; ++i) {
            if (text[i] == '\\' && i + 1 < text.size()) ++i;
            value += text[i];
        }
        out.push_back(value);
    }
    return out;
}

}  // namespace detail

class MACEKokkosFloat {
public:
    // MACEKokkos(std::string filename, std::string requested_head = {})
    explicit MACEKokkosFloat(const std::string& filename, const std::string& requested_head = {})
    {
        detail::check(sxl_create(filename.c_str(), requested_head.c_str(), &handle_));
        sxl_model_info_t info{};
        detail::check(sxl_model_info(handle_, &info));
        r_cut = info.r_cut;
        l_max = info.l_max;
        num_lm = (l_max + 1) * (l_max + 1);
        L_max = info.L_max;
        num_LM = (L_max + 1) * (L_max + 1);
        num_channels = info.num_channels;
        atomic_numbers_host.resize(static_cast<std::size_t>(info.num_elements));
        atomic_energies.resize(static_cast<std::size_t>(info.num_elements));
        detail::check(sxl_atomic_numbers(handle_, atomic_numbers_host.data()));
        detail::check(sxl_atomic_energies(handle_, atomic_energies.data()));
        const std::string heads = detail::json_text([this](char* b, std::int64_t c, std::int64_t* n) {
            return sxl_model_heads_json(handle_, b, c, n);
        });
        // {"selected_head": "...", "available_heads": [...]}
        const std::size_t list = heads.find('[');
        const std::vector<std::string> first = detail::json_strings(heads, 0, list);
        selected_head = first.size() >= 2 ? first[1] : std::string();
        available_heads = detail::json_strings(heads, list, heads.find(']', list));
    }

    ~MACEKokkosFloat() { sxl_destroy(handle_); }
    MACEKokkosFloat(const MACEKokkosFloat&) = delete;
    MACEKokkosFloat& operator=(const MACEKokkosFloat&) = delete;
    MACEKokkosFloat(MACEKokkosFloat&& other) noexcept { swap(other); }
    MACEKokkosFloat& operator=(MACEKokkosFloat&& other) noexcept
    {
        swap(other);
        return *this;
    }

    // model properties (public members of the reference)
    double r_cut = 0.0;
    int l_max = 0, num_lm = 0;
    int L_max = 0, num_LM = 0;
    int num_channels = 0;
    std::vector<int> atomic_numbers_host;
    std::vector<double> atomic_energies;
    std::string selected_head;
    std::vector<std::string> available_heads;

    // prepare_factorized_graph(num_nodes, node_types, num_neigh, neigh_indices, neigh_types)
    std::uint64_t prepare_factorized_graph(int num_nodes, std::span<const int> node_types,
                                           std::span<const int> num_neigh, std::span<const int> neigh_indices,
                                           std::span<const int> neigh_types)
    {
        detail::require(num_nodes >= 0 && node_types.size() == static_cast<std::size_t>(num_nodes) &&
                            num_neigh.size() == static_cast<std::size_t>(num_nodes),
                        "Factorized graph node arrays must hold num_nodes entries.");
        detail::require(neigh_indices.size() == neigh_types.size(),
                        "Factorized graph neighbour arrays have different extents.");
        std::uint64_t generation = 0;
        detail::check(sxl_prepare_graph(handle_, num_nodes, node_types.data(), num_neigh.data(),
                                        neigh_indices.data(), neigh_types.data(), &generation));
        return generation;
    }

    // the same from device arrays (the reference's Kokkos::View overload,
    // mace_kokkos.hpp:339-460): node_types, num_neigh [num_nodes],
    // neigh_indices, neigh_types [sum of num_neigh] in device memory
    std::uint64_t prepare_factorized_graph_device(int num_nodes, const int* d_node_types, const int* d_num_neigh,
                                                  const int* d_neigh_indices, const int* d_neigh_types)
    {
        detail::require(num_nodes >= 0, "num_nodes must be non-negative.");
        std::uint64_t generation = 0;
        detail::check(sxl_prepare_graph_device(handle_, num_nodes, d_node_types, d_num_neigh, d_neigh_indices,
                                               d_neigh_types, &generation));
        return generation;
    }

    // prepare_periodic_factorized_graph(node_types, positions, cell, inverse_cell, neighbor_cutoff)
    //   -> {generation, num_edges}
    std::pair<std::uint64_t, std::size_t> prepare_periodic_factorized_graph(std::span<const int> node_types,
                                                                            std::span<const double> positions,
                                                                            std::span<const double> cell,
                                                                            std::span<const double> inverse_cell,
                                                                            double neighbor_cutoff)
    {
        detail::require(positions.size() == 3 * node_types.size(), "positions must hold 3 * num_nodes values.");
        detail::require(cell.size() == 9 && inverse_cell.size() == 9, "cell and inverse_cell must hold 9 values.");
        std::uint64_t generation = 0;
        std::int64_t edges = 0;
        detail::check(sxl_prepare_periodic_graph(handle_, static_cast<int>(node_types.size()), node_types.data(),
                                                 positions.data(), cell.data(), inverse_cell.data(),
                                                 neighbor_cutoff, &generation, &edges));
        return {generation, static_cast<std::size_t>(edges)};
    }

    // update_factorized_cell(graph_generation, cell, inverse_cell)
    void update_factorized_cell(std::uint64_t graph_generation, std::span<const double> cell,
                                std::span<const double> inverse_cell)
    {
        detail::require(cell.size() == 9 && inverse_cell.size() == 9, "cell and inverse_cell must hold 9 values.");
        detail::check(sxl_update_cell(handle_, graph_generation, cell.data(), inverse_cell.data()));
    }

    // validate_graph_cardinality(num_receivers, num_feature_nodes, num_edges)
    void validate_graph_cardinality(std::size_t num_receivers, std::size_t num_feature_nodes,
                                    std::size_t num_edges) const
    {
        detail::check(sxl_validate_graph_cardinality(handle_, static_cast<std::int64_t>(num_receivers),
                                                     static_cast<std::int64_t>(num_feature_nodes),
                                                     static_cast<std::int64_t>(num_edges)));
    }

    // prepare_factorized_geometry(graph_generation, reference_positions,
    // reference_xyz, cell, inverse_cell, pbc)
    void prepare_factorized_geometry(std::uint64_t graph_generation, std::span<const double> reference_positions,
                                     std::span<const double> reference_xyz, std::span<const double> cell,
                                     std::span<const double> inverse_cell, std::span<const int> pbc)
    {
        detail::require(cell.size() == 9 && inverse_cell.size() == 9 && pbc.size() == 3,
                        "Execution R1 prepared geometry extents are inconsistent.");
        detail::check(sxl_prepare_geometry(handle_, graph_generation, reference_positions.data(),
                                           static_cast<std::int64_t>(reference_positions.size()),
                                           reference_xyz.data(), static_cast<std::int64_t>(reference_xyz.size()),
                                           cell.data(), inverse_cell.data(), pbc.data()));
    }

    // prepare_factorized_fractional_geometry(graph_generation,
    // fractional_positions, fractional_xyz, cell, inverse_cell, pbc)
    void prepare_factorized_fractional_geometry(std::uint64_t graph_generation,
                                                std::span<const double> fractional_positions,
                                                std::span<const double> fractional_xyz, std::span<const double> cell,
                                                std::span<const double> inverse_cell, std::span<const int> pbc)
    {
        detail::require(cell.size() == 9 && inverse_cell.size() == 9 && pbc.size() == 3,
                        "Fractional Execution R1 geometry requires 3x3 cell matrices and three PBC flags.");
        detail::check(sxl_prepare_fractional_geometry(
            handle_, graph_generation, fractional_positions.data(),
            static_cast<std::int64_t>(fractional_positions.size()), fractional_xyz.data(),
            static_cast<std::int64_t>(fractional_xyz.size()), cell.data(), inverse_cell.data(), pbc.data()));
    }

    // prepare_factorized_shift_geometry(graph_generation, reference_positions,
    // shifts, cell, inverse_cell, pbc)
    void prepare_factorized_shift_geometry(std::uint64_t graph_generation,
                                           std::span<const double> reference_positions, std::span<const int> shifts,
                                           std::span<const double> cell, std::span<const double> inverse_cell,
                                           std::span<const int> pbc)
    {
        detail::require(cell.size() == 9 && inverse_cell.size() == 9 && pbc.size() == 3,
                        "Shift geometry extents are inconsistent.");
        detail::check(sxl_prepare_shift_geometry(handle_, graph_generation, reference_positions.data(),
                                                 static_cast<std::int64_t>(reference_positions.size()),
                                                 shifts.data(), static_cast<std::int64_t>(shifts.size()),
                                                 cell.data(), inverse_cell.data(), pbc.data()));
    }

    // compute_prepared_factorized(graph_generation, xyz, r)
    void compute_prepared_factorized(std::uint64_t graph_generation, std::span<const double> xyz,
                                     std::span<const double> r)
    {
        const std::size_t edges = num_edges();
        detail::require(xyz.size() == 3 * edges && r.size() == edges,
                        "xyz and r must hold 3 * num_edges and num_edges values.");
        detail::check(sxl_compute_prepared(handle_, graph_generation, xyz.data(), r.data()));
        evaluated(graph_generation);
    }

    // compute_prepared_factorized_positions(graph_generation, positions)
    void compute_prepared_factorized_positions(std::uint64_t graph_generation, std::span<const double> positions)
    {
        detail::require(positions.size() == 3 * static_cast<std::size_t>(num_nodes()),
                        "positions must hold 3 * num_nodes values.");
        detail::check(sxl_compute_prepared_positions(handle_, graph_generation, positions.data()));
        evaluated(graph_generation);
    }

    // the same two evaluations from device arrays: xyz [3 E], r [E] or
    // positions [3 N] in device memory (results stay on the device until read)
    void compute_prepared_factorized_device(std::uint64_t graph_generation, const double* d_xyz, const double* d_r)
    {
        detail::check(sxl_compute_prepared_device(handle_, graph_generation, d_xyz, d_r));
        evaluated(graph_generation);
    }
    void compute_prepared_factorized_positions_device(std::uint64_t graph_generation, const double* d_positions)
    {
        detail::check(sxl_compute_prepared_positions_device(handle_, graph_generation, d_positions));
        evaluated(graph_generation);
    }

    // compute_node_energies_forces(num_nodes, node_types, num_neigh, neigh_indices,
    //                              neigh_types, xyz, r, execution_graph_generation = 0)
    void compute_node_energies_forces(int num_nodes, std::span<const int> node_types, std::span<const int> num_neigh,
                                      std::span<const int> neigh_indices, std::span<const int> neigh_types,
                                      std::span<const double> xyz, std::span<const double> r,
                                      std::uint64_t execution_graph_generation = 0)
    {
        if (execution_graph_generation != 0) {
            compute_prepared_factorized(execution_graph_generation, xyz, r);
            return;
        }
        detail::require(num_nodes >= 0 && node_types.size() == static_cast<std::size_t>(num_nodes) &&
                            num_neigh.size() == static_cast<std::size_t>(num_nodes),
                        "Node arrays must hold num_nodes entries.");
        detail::require(neigh_types.size() == neigh_indices.size() && r.size() == neigh_indices.size() &&
                            xyz.size() == 3 * neigh_indices.size(),
                        "Edge arrays have inconsistent extents.");
        detail::check(sxl_compute_node_energies_forces(handle_, num_nodes, node_types.data(), num_neigh.data(),
                                                       neigh_indices.data(), neigh_types.data(), xyz.data(),
                                                       r.data()));
        evaluated(generation());
    }

    // reduce_prepared_node_forces(graph_generation): atom_forces() = sum of the
    // directed forces per atom
    void reduce_prepared_node_forces(std::uint64_t graph_generation)
    {
        atom_forces_.assign(3 * static_cast<std::size_t>(num_nodes()), 0.0);
        detail::check(sxl_reduce_atom_forces(handle_, graph_generation, atom_forces_.data()));
    }

    // reduce_prepared_stress(volume, graph_generation): stress_tensor() (3 x 3, row-major)
    void reduce_prepared_stress(double volume, std::uint64_t graph_generation)
    {
        stress_tensor_.assign(9, 0.0);
        detail::check(sxl_reduce_stress(handle_, graph_generation, volume, stress_tensor_.data()));
    }

    // set_execution_plan_request(algorithm, profile, debug_plan = {})
    void set_execution_plan_request(std::string algorithm, std::string profile, std::string debug_plan = {})
    {
        detail::check(sxl_set_execution_plan_request(handle_, algorithm.c_str(), profile.c_str(),
                                                     debug_plan.c_str()));
    }

    // execution_plan_report() as the JSON object the Python binding returns
    std::string execution_plan_report_json() const
    {
        return detail::json_text([this](char* b, std::int64_t c, std::int64_t* n) {
            return sxl_execution_plan_json(handle_, b, c, n);
        });
    }

    // device memory by role and the plan's capacities (sxl_workspace_json)
    std::string workspace_json() const
    {
        return detail::json_text([this](char* b, std::int64_t c, std::int64_t* n) {
            return sxl_workspace_json(handle_, b, c, n);
        });
    }

    // set_allow_fixed_workspace(bool)
    void set_allow_fixed_workspace(bool allow) { detail::check(sxl_set_allow_fixed_workspace(handle_, allow ? 1 : 0)); }

    // results of the last evaluation (host copies)
    const std::vector<double>& node_energies()
    {
        if (!energies_fresh_) {
            node_energies_.assign(static_cast<std::size_t>(num_nodes()), 0.0);
            detail::check(sxl_node_energies(handle_, node_energies_.data(), num_nodes()));
            energies_fresh_ = true;
        }
        return node_energies_;
    }

    // directed forces f_ij = -dE/dxyz_ij, 3 per edge
    const std::vector<double>& node_forces()
    {
        if (!forces_fresh_) {
            const std::size_t edges = num_edges();
            node_forces_.assign(3 * edges, 0.0);
            detail::check(sxl_node_forces(handle_, node_forces_.data(), static_cast<std::int64_t>(edges)));
            forces_fresh_ = true;
        }
        return node_forces_;
    }

    const std::vector<double>& atom_forces() const { return atom_forces_; }
    const std::vector<double>& stress_tensor() const { return stress_tensor_; }

    // sum of the node energies of the last evaluation on graph_generation
    double total_energy(std::uint64_t graph_generation)
    {
        double e = 0.0;
        detail::check(sxl_total_energy(handle_, graph_generation, &e));
        return e;
    }

    int num_nodes() const
    {
        int n = 0;
        std::int64_t e = 0;
        std::uint64_t g = 0;
        detail::check(sxl_graph_size(handle_, &n, &e, &g));
        return n;
    }

    std::size_t num_edges() const
    {
        int n = 0;
        std::int64_t e = 0;
        std::uint64_t g = 0;
        detail::check(sxl_graph_size(handle_, &n, &e, &g));
        return static_cast<std::size_t>(e);
    }

    // generation token of the prepared graph (0: none)
    std::uint64_t generation() const
    {
        int n = 0;
        std::int64_t e = 0;
        std::uint64_t g = 0;
        detail::check(sxl_graph_size(handle_, &n, &e, &g));
        return g;
    }

    // the C handle, for the functions of symmetrix_amd.h without a method here
    sxl_evaluator* handle() const { return handle_; }

private:
    void evaluated(std::uint64_t)
    {
        energies_fresh_ = false;
        forces_fresh_ = false;
    }

    void swap(MACEKokkosFloat& o) noexcept
    {
        std::swap(handle_, o.handle_);
        std::swap(r_cut, o.r_cut);
        std::swap(l_max, o.l_max);
        std::swap(num_lm, o.num_lm);
        std::swap(L_max, o.L_max);
        std::swap(num_LM, o.num_LM);
        std::swap(num_channels, o.num_channels);
        atomic_numbers_host.swap(o.atomic_numbers_host);
        atomic_energies.swap(o.atomic_energies);
        selected_head.swap(o.selected_head);
        available_heads.swap(o.available_heads);
        node_energies_.swap(o.node_energies_);
        node_forces_.swap(o.node_forces_);
        atom_forces_.swap(o.atom_forces_);
        stress_tensor_.swap(o.stress_tensor_);
        std::swap(energies_fresh_, o.energies_fresh_);
        std::swap(forces_fresh_, o.forces_fresh_);
    }

    sxl_evaluator* handle_ = nullptr;
    std::vector<double> node_energies_, node_forces_, atom_forces_, stress_tensor_;
    bool energies_fresh_ = false, forces_fresh_ = false;
};

}  // namespace symmetrix_amd
