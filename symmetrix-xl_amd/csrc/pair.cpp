// Single-rank pair-style driver (see pair.hpp).
#include "pair.hpp"

#include <cmath>
#include <limits>
#include <stdexcept>
#include <string>

#include "kernels.hpp"

// the host entry forms edge vectors and lengths as the device entry's kernel
// does (no fused operations), so both evaluate the same inputs
#pragma clang fp contract(off)

namespace sxl {

namespace {
void hip_check(hipError_t err, const char* what)
{
    if (err != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(err));
}
}  // namespace

void PairDriver::check_types(const Evaluator& ev, int ntypes, const int* mace_types) const
{
    const HostModel& model = ev.model();
    for (int t = 0; t < ntypes; ++t)
        if (mace_types[t] < 0 || mace_types[t] >= model.num_elements)
            throw std::invalid_argument("pair_coeff maps a LAMMPS type to an element outside the model");
}

// The LAMMPS virial sum xyz (x) f from the evaluator's stress reduction at
// unit volume (-sum f (x) xyz), and the energy from its node-energy sum.
void PairDriver::totals(Evaluator& ev, std::uint64_t g, const PairOutput& out)
{
    if (out.energy) *out.energy += ev.total_energy(g);
    if (out.virial) {
        double s[9];
        ev.stress(g, 1.0, s);
        out.virial[0] -= s[0];
        out.virial[1] -= s[4];
        out.virial[2] -= s[8];
        out.virial[3] -= 0.5 * (s[1] + s[3]);
        out.virial[4] -= 0.5 * (s[2] + s[6]);
        out.virial[5] -= 0.5 * (s[5] + s[7]);
    }
}

void PairDriver::compute(Evaluator& ev, const PairInput& in, const PairOutput& out)
{
    if (in.inum < 0 || in.nall < in.inum) throw std::invalid_argument("pair list has invalid atom counts");
    if (!out.f) throw std::invalid_argument("pair compute requires a force array");
    if (in.inum == 0) return;
    if (!in.ilist || !in.numneigh || !in.firstneigh || !in.x || !in.type || !in.local_of || !in.mace_types)
        throw std::invalid_argument("pair list arrays must not be null");
    check_types(ev, in.ntypes, in.mace_types);
    auto element = [&](int atom) {
        const int t = in.type[atom];
        if (t < 1 || t > in.ntypes) throw std::out_of_range("LAMMPS atom type out of range");
        return in.mace_types[t - 1];
    };
    const double rc2 = ev.model().r_cut * ev.model().r_cut;
    const int n = in.inum;

    // ii_from_i: position of each local atom in ilist
    ii_from_i_.assign(in.nall, -1);
    for (int ii = 0; ii < n; ++ii) {
        const int i = in.ilist[ii];
        if (i < 0 || i >= in.nall || ii_from_i_[i] >= 0)
            throw std::out_of_range("ilist holds an atom index out of range or twice");
        ii_from_i_[i] = ii;
    }

    node_types_.resize(n);
    num_neigh_.assign(n, 0);
    node_i_.resize(n);
    neigh_indices_.clear();
    neigh_types_.clear();
    xyz_.clear();
    r_.clear();
    for (int ii = 0; ii < n; ++ii) {
        const int i = in.ilist[ii];
        node_i_[ii] = i;
        node_types_[ii] = element(i);
        const double* xi = in.x + 3 * static_cast<std::size_t>(i);
        const int* jlist = in.firstneigh[i];
        const int count = in.numneigh[i];
        if (count < 0 || (count > 0 && !jlist)) throw std::invalid_argument("neighbour list of an atom is invalid");
        for (int jj = 0; jj < count; ++jj) {
            const int j = jlist[jj] & kNeighMask;
            if (j < 0 || j >= in.nall) throw std::out_of_range("neighbour index out of range");
            const double* xj = in.x + 3 * static_cast<std::size_t>(j);
            const double dx = xj[0] - xi[0], dy = xj[1] - xi[1], dz = xj[2] - xi[2];
            const double r2 = dx * dx + dy * dy + dz * dz;
            if (!(r2 < rc2)) continue;
            const int j_local = in.local_of[j];
            if (j_local < 0 || j_local >= in.nall || ii_from_i_[j_local] < 0)
                throw std::invalid_argument("a neighbour maps to an atom that is not in the local list");
            num_neigh_[ii] += 1;
            neigh_indices_.push_back(ii_from_i_[j_local]);
            neigh_types_.push_back(element(j));
            xyz_.push_back(dx);
            xyz_.push_back(dy);
            xyz_.push_back(dz);
            r_.push_back(std::sqrt(r2));
        }
    }

    const std::uint64_t g =
        ev.prepare_graph(n, node_types_.data(), num_neigh_.data(), neigh_indices_.data(), neigh_types_.data());
    ev.compute_xyz(g, xyz_.data(), r_.data(), false);
    node_forces_.resize(3 * static_cast<std::size_t>(n));
    ev.atom_forces(g, node_forces_.data());
    for (int ii = 0; ii < n; ++ii)
        for (int c = 0; c < 3; ++c) out.f[3 * static_cast<std::size_t>(node_i_[ii]) + c] += node_forces_[3 * ii + c];
    if (out.eatom) {
        node_energies_.resize(n);
        ev.node_energies(node_energies_.data());
        for (int ii = 0; ii < n; ++ii) out.eatom[node_i_[ii]] = node_energies_[ii];
    }
    totals(ev, g, out);
}

// The list as a PairList over the device arrays (mace_types copied to the
// device on the evaluator's stream).
PairList PairDriver::device_list(Evaluator& ev, const PairDeviceInput& in, bool stable)
{
    if (in.inum < 0 || in.nall < in.inum) throw std::invalid_argument("pair list has invalid atom counts");
    if (!in.ilist || !in.numneigh || !in.neighbors || !in.x || !in.type || !in.local_of || !in.mace_types)
        throw std::invalid_argument("pair list arrays must not be null");
    if (in.ntypes < 1) throw std::invalid_argument("pair compute requires the pair_coeff type map");
    check_types(ev, in.ntypes, in.mace_types);
    std::vector<int> map(in.mace_types, in.mace_types + in.ntypes);
    d_mace_types_.reserve(map.size() * sizeof(int));
    hip_check(hipMemcpyAsync(d_mace_types_.as<int>(), map.data(), map.size() * sizeof(int), hipMemcpyHostToDevice,
                             ev.stream()),
              "type map");
    PairList p;
    p.inum = in.inum;
    p.ilist = in.ilist;
    p.numneigh = in.numneigh;
    p.neighbors = in.neighbors;
    p.stride_atom = in.stride_atom;
    p.stride_slot = in.stride_slot;
    p.nall = in.nall;
    p.x = in.x;
    p.type = in.type;
    p.local_of = in.local_of;
    p.ntypes = in.ntypes;
    p.mace_types = d_mace_types_.as<int>();
    p.r_cut_squared = ev.model().r_cut * ev.model().r_cut;
    p.r_cut = ev.model().r_cut;
    p.stable = stable ? 1 : 0;
    return p;
}

// Filters and maps the list on the device and prepares its graph: the
// per-atom neighbour counts come to the host once.  Leaves the edge vectors
// in d_xyz_ / d_r_ and returns the graph's generation.
std::uint64_t PairDriver::prepare_device_graph(Evaluator& ev, const PairList& p)
{
    hipStream_t s = ev.stream();
    const int n = p.inum;
    d_ii_from_i_.reserve(static_cast<std::size_t>(p.nall) * sizeof(int));
    d_node_types_.reserve(static_cast<std::size_t>(n) * sizeof(int));
    d_num_neigh_.reserve(static_cast<std::size_t>(n) * sizeof(int));
    d_offsets_.reserve((static_cast<std::size_t>(n) + 1) * sizeof(long long));
    d_flags_.reserve(sizeof(unsigned));
    hip_check(hipMemsetAsync(d_flags_.as<void>(), 0, sizeof(unsigned), s), "memset");
    hip_check(launch_fill_i32(d_ii_from_i_.as<int>(), p.nall, -1, s), "list index");
    hip_check(launch_pair_index(n, p.ilist, p.nall, d_ii_from_i_.as<int>(), d_flags_.as<unsigned>(), s), "list index");
    hip_check(launch_pair_edges(p, d_ii_from_i_.as<int>(), nullptr, d_node_types_.as<int>(), d_num_neigh_.as<int>(),
                                nullptr, nullptr, nullptr, nullptr, d_flags_.as<unsigned>(), s),
              "list count");
    num_neigh_.resize(n);
    unsigned flags = 0;
    hip_check(hipMemcpyAsync(num_neigh_.data(), d_num_neigh_.as<int>(), n * sizeof(int), hipMemcpyDeviceToHost, s),
              "copy");
    hip_check(hipMemcpyAsync(&flags, d_flags_.as<void>(), sizeof(unsigned), hipMemcpyDeviceToHost, s), "copy");
    hip_check(host_fence(s), "list count");
    if (flags & 1u) throw std::out_of_range("ilist holds an atom index out of range or twice");
    if (flags & 2u) throw std::out_of_range("neighbour index out of range");
    if (flags & 4u) throw std::out_of_range("LAMMPS atom type out of range");
    if (flags & 8u) throw std::invalid_argument("a neighbour maps to an atom that is not in the local list");
    std::vector<long long> offsets(static_cast<std::size_t>(n) + 1, 0);
    for (int ii = 0; ii < n; ++ii) offsets[ii + 1] = offsets[ii] + num_neigh_[ii];
    const long long E = offsets[n];
    if (E > std::numeric_limits<int>::max())
        throw std::length_error("MACE graph directed-edge count exceeds the 32-bit topology limit.");
    hip_check(hipMemcpyAsync(d_offsets_.as<long long>(), offsets.data(), offsets.size() * sizeof(long long),
                             hipMemcpyHostToDevice, s),
              "offsets");
    const std::size_t Es = static_cast<std::size_t>(std::max<long long>(E, 1));
    d_neigh_indices_.reserve(Es * sizeof(int));
    d_neigh_types_.reserve(Es * sizeof(int));
    d_xyz_.reserve(Es * 3 * sizeof(double));
    d_r_.reserve(Es * sizeof(double));
    hip_check(launch_pair_edges(p, d_ii_from_i_.as<int>(), d_offsets_.as<long long>(), nullptr, nullptr,
                                d_neigh_indices_.as<int>(), d_neigh_types_.as<int>(), d_xyz_.as<double>(),
                                d_r_.as<double>(), nullptr, s),
              "list edges");
    // prepare_graph_device waits on the stream, so the host offsets outlive their copy
    const std::uint64_t g = ev.prepare_graph_device(n, d_node_types_.as<int>(), d_num_neigh_.as<int>(),
                                                    d_neigh_indices_.as<int>(), d_neigh_types_.as<int>());
    return g;
}

// Evaluates the graph g on the edge vectors in d_xyz_ / d_r_ and adds the
// results to the pair style's accumulators.
void PairDriver::evaluate_device(Evaluator& ev, std::uint64_t g, const PairDeviceInput& in, const PairOutput& out)
{
    ev.compute_xyz(g, d_xyz_.as<double>(), d_r_.as<double>(), true);
    hip_check(launch_pair_scatter(in.inum, in.ilist, ev.device_atom_forces(), ev.device_node_energies(), out.f,
                                  out.eatom, ev.stream()),
              "pair forces");
    totals(ev, g, out);
    ev.synchronize();  // the forces and energies are in place on return
}

void PairDriver::compute_device(Evaluator& ev, const PairDeviceInput& in, const PairOutput& out)
{
    if (in.inum < 0 || in.nall < in.inum) throw std::invalid_argument("pair list has invalid atom counts");
    if (!out.f) throw std::invalid_argument("pair compute requires a force array");
    if (in.inum == 0) return;
    const PairList p = device_list(ev, in, false);
    const std::uint64_t g = prepare_device_graph(ev, p);
    prepared_generation_ = 0;  // the stable entry's graph is replaced
    evaluate_device(ev, g, in, out);
}

void PairDriver::compute_device_prepared(Evaluator& ev, int neighbor_ago, const PairDeviceInput& in,
                                         const PairOutput& out, bool* rebuilt)
{
    if (rebuilt) *rebuilt = false;
    if (in.inum < 0 || in.nall < in.inum) throw std::invalid_argument("pair list has invalid atom counts");
    if (!out.f) throw std::invalid_argument("pair compute requires a force array");
    if (in.inum == 0) return;
    const PairList p = device_list(ev, in, true);
    const bool rebuild = neighbor_ago == 0 || prepared_generation_ == 0 || ev.generation() != prepared_generation_ ||
                         in.inum != prepared_inum_ || in.nall != prepared_nall_;
    if (rebuild) {
        prepared_generation_ = 0;
        const std::uint64_t g = prepare_device_graph(ev, p);
        prepared_generation_ = g;
        prepared_inum_ = in.inum;
        prepared_nall_ = in.nall;
        ++graph_rebuilds_;
        if (rebuilt) *rebuilt = true;
    } else {
        // an unchanged list (LAMMPS neighbor->ago > 0): only the edge vectors
        hipStream_t s = ev.stream();
        hip_check(hipMemsetAsync(d_flags_.as<void>(), 0, sizeof(unsigned), s), "memset");
        hip_check(launch_pair_edges(p, nullptr, d_offsets_.as<long long>(), nullptr, nullptr, nullptr, nullptr,
                                    d_xyz_.as<double>(), d_r_.as<double>(), d_flags_.as<unsigned>(), s),
                  "list geometry");
        flags_host_.reserve(sizeof(unsigned));
        hip_check(hipMemcpyAsync(flags_host_.as<unsigned>(), d_flags_.as<void>(), sizeof(unsigned),
                                 hipMemcpyDeviceToHost, s),
                  "copy");
        ++geometry_updates_;
    }
    evaluate_device(ev, prepared_generation_, in, out);
    if (!rebuild && *flags_host_.as<unsigned>() != 0) {
        prepared_generation_ = 0;
        throw std::invalid_argument(
            "the neighbour list changed without a rebuild (neighbor_ago > 0 requires the list of the last call)");
    }
}

}  // namespace sxl
