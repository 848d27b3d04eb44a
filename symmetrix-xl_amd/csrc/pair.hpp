// Single-rank LAMMPS pair-style driver over the evaluator: the counterpart of
// PairSymmetrixMACE::compute_no_domain_decomposition
// (pair_symmetrix/pair_symmetrix_mace.cpp:309-441).  A LAMMPS full neighbour
// list over local and ghost atoms is filtered to r < r_cut, ghosts are mapped
// to their local atoms (atom->map(atom->tag[j])), the receiver-major graph is
// evaluated on the device, and the directed edge forces are folded into the
// local atoms' forces and the global virial.
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

struct PairOutput {
    double* f = nullptr;       // [nall][3], accumulated
    double* energy = nullptr;  // global energy, accumulated (may be null)
    double* eatom = nullptr;   // [nall] per-atom energy, set for local atoms (may be null)
    double* virial = nullptr;  // [6] xx yy zz xy xz yz, accumulated (may be null)
};

class PairDriver {
public:
    void compute(Evaluator& ev, const PairInput& in, const PairOutput& out);

private:
    std::vector<int> ii_from_i_, node_types_, num_neigh_, neigh_indices_, neigh_types_, node_i_, neigh_j_;
    std::vector<double> xyz_, r_, node_energies_, node_forces_;
};

}  // namespace sxl
