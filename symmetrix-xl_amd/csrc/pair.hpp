// Single-rank LAMMPS pair-style driver over the evaluator: the counterpart of
// PairSymmetrixMACE::compute_no_domain_decomposition
// (pair_symmetrix/pair_symmetrix_mace.cpp:309-441) and, on device arrays, of
// PairSymmetrixMACEKokkos::compute_no_domain_decomposition
// (pair_symmetrix/pair_symmetrix_mace_kokkos.cpp:1010-1260).  A LAMMPS full
// neighbour list over local and ghost atoms is filtered to r < r_cut, ghosts
// are mapped to their local atoms (atom->map(atom->tag[j])), the
// receiver-major graph is evaluated on the device, and its reduced node
// forces (the sum of each atom's outgoing minus incoming directed forces),
// energy and virial are added to the pair style's accumulators.  Both entries
// use the same device reductions, so they give the same results bit for bit.
#pragma once

#include <vector>

#include "evaluator.hpp"

namespace sxl {

// LAMMPS neighbour-list bits above NEIGHMASK flag special bonds
constexpr int kNeighMask = 0x1FFFFFFF;

struct PairInput {
    int inum = 0;                          // local atoms in the list
    const int* ilist = nullptr;            // [inum] atom indices
    const int* numneigh = nullptr;         // [nall] indexed by atom
    const int* const* firstneigh = nullptr;  // [nall] per-atom neighbour arrays (masked by kNeighMask)
    int nall = 0;                          // local + ghost atoms
    const double* x = nullptr;             // [nall][3]
    const int* type = nullptr;             // [nall] LAMMPS types, 1-based
    const int* local_of = nullptr;         // [nall] local atom of each atom (atom->map(atom->tag[j]))
    int ntypes = 0;
    const int* mace_types = nullptr;       // [ntypes] model element index of LAMMPS type t + 1
};

// The same list in device memory (a LAMMPS KOKKOS list): neighbour slot jj
// of atom i at neighbors[i stride_atom + jj stride_slot]; mace_types stays a
// host array.
struct PairDeviceInput {
    int inum = 0;
    const int* ilist = nullptr;
    const int* numneigh = nullptr;
    const int* neighbors = nullptr;
    long long stride_atom = 0, stride_slot = 1;
    int nall = 0;
    const double* x = nullptr;
    const int* type = nullptr;
    const int* local_of = nullptr;
    int ntypes = 0;
    const int* mace_types = nullptr;
};

struct PairOutput {
    double* f = nullptr;       // [nall][3], accumulated (device memory for the device entry)
    double* energy = nullptr;  // global energy, accumulated (host, may be null)
    double* eatom = nullptr;   // [nall] per-atom energy, set for local atoms (may be null; device for the device entry)
    double* virial = nullptr;  // [6] xx yy zz xy xz yz, accumulated (host, may be null)
};

class PairDriver {
public:
    void compute(Evaluator& ev, const PairInput& in, const PairOutput& out);
    void compute_device(Evaluator& ev, const PairDeviceInput& in, const PairOutput& out);
    // The reference Kokkos pair style's prepared execution
    // (pair_symmetrix_mace_kokkos.cpp:1043-1160): every listed pair is an
    // edge (those at r >= r_cut scaled to length r_cut, contributing
    // nothing), and while the list is unchanged (neighbor_ago > 0, same atom
    // counts, the evaluator still on this graph) only the edge vectors are
    // updated and the prepared graph is evaluated again.
    void compute_device_prepared(Evaluator& ev, int neighbor_ago, const PairDeviceInput& in, const PairOutput& out,
                                 bool* rebuilt);
    long long graph_rebuilds() const { return graph_rebuilds_; }
    long long geometry_updates() const { return geometry_updates_; }

private:
    void check_types(const Evaluator& ev, int ntypes, const int* mace_types) const;
    // energy and virial of the evaluated graph into the host accumulators
    void totals(Evaluator& ev, std::uint64_t generation, const PairOutput& out);
    PairList device_list(Evaluator& ev, const PairDeviceInput& in, bool stable);
    std::uint64_t prepare_device_graph(Evaluator& ev, const PairList& p);
    void evaluate_device(Evaluator& ev, std::uint64_t generation, const PairDeviceInput& in, const PairOutput& out);
    std::uint64_t prepared_generation_ = 0;
    int prepared_inum_ = 0, prepared_nall_ = 0;
    long long graph_rebuilds_ = 0, geometry_updates_ = 0;
    PinnedBuffer flags_host_;
    std::vector<int> ii_from_i_, node_types_, num_neigh_, neigh_indices_, neigh_types_, node_i_;
    std::vector<double> xyz_, r_, node_energies_, node_forces_;
    // device entry
    DeviceBuffer d_mace_types_, d_ii_from_i_, d_node_types_, d_num_neigh_, d_offsets_, d_neigh_indices_,
        d_neigh_types_, d_xyz_, d_r_, d_flags_;
};

}  // namespace sxl
