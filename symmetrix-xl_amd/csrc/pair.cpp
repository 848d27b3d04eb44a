// Single-rank pair-style driver (see pair.hpp).
#include "pair.hpp"

#include <cmath>
#include <stdexcept>
#include <string>

namespace sxl {

void PairDriver::compute(Evaluator& ev, const PairInput& in, const PairOutput& out)
{
    if (in.inum < 0 || in.nall < in.inum) throw std::invalid_argument("pair list has invalid atom counts");
    if (!out.f) throw std::invalid_argument("pair compute requires a force array");
    if (in.inum == 0) return;
    if (!in.ilist || !in.numneigh || !in.firstneigh || !in.x || !in.type || !in.local_of || !in.mace_types)
        throw std::invalid_argument("pair list arrays must not be null");
    const HostModel& model = ev.model();
    for (int t = 0; t < in.ntypes; ++t)
        if (in.mace_types[t] < 0 || in.mace_types[t] >= model.num_elements)
            throw std::invalid_argument("pair_coeff maps a LAMMPS type to an element outside the model");
    auto element = [&](int atom) {
        const int t = in.type[atom];
        if (t < 1 || t > in.ntypes) throw std::out_of_range("LAMMPS atom type out of range");
        return in.mace_types[t - 1];
    };
    const double rc2 = model.r_cut * model.r_cut;
    const int n = in.inum;

    // ii_from_i: position of each local atom in ilist
    ii_from_i_.assign(in.nall, -1);
    for (int ii = 0; ii < n; ++ii) {
        const int i = in.ilist[ii];
        if (i < 0 || i >= in.nall) throw std::out_of_range("ilist holds an atom index out of range");
        ii_from_i_[i] = ii;
    }

    node_types_.resize(n);
    num_neigh_.assign(n, 0);
    node_i_.resize(n);
    neigh_indices_.clear();
    neigh_types_.clear();
    neigh_j_.clear();
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
            neigh_j_.push_back(j_local);
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
    const std::size_t E = r_.size();
    node_energies_.resize(n);
    node_forces_.resize(3 * E);
    ev.node_energies(node_energies_.data());
    if (E > 0) ev.node_forces(node_forces_.data());

    if (out.energy)
        for (int ii = 0; ii < n; ++ii) *out.energy += node_energies_[ii];
    if (out.eatom)
        for (int ii = 0; ii < n; ++ii) out.eatom[node_i_[ii]] = node_energies_[ii];
    std::size_t ij = 0;
    for (int ii = 0; ii < n; ++ii) {
        double* fi = out.f + 3 * static_cast<std::size_t>(node_i_[ii]);
        for (int jj = 0; jj < num_neigh_[ii]; ++jj, ++ij) {
            double* fj = out.f + 3 * static_cast<std::size_t>(neigh_j_[ij]);
            for (int c = 0; c < 3; ++c) {
                fi[c] -= node_forces_[3 * ij + c];
                fj[c] += node_forces_[3 * ij + c];
            }
        }
    }
    if (out.virial)
        for (std::size_t e = 0; e < E; ++e) {
            const double x = xyz_[3 * e], y = xyz_[3 * e + 1], z = xyz_[3 * e + 2];
            const double fx = node_forces_[3 * e], fy = node_forces_[3 * e + 1], fz = node_forces_[3 * e + 2];
            out.virial[0] += x * fx;
            out.virial[1] += y * fy;
            out.virial[2] += z * fz;
            out.virial[3] += 0.5 * (x * fy + y * fx);
            out.virial[4] += 0.5 * (x * fz + z * fx);
            out.virial[5] += 0.5 * (y * fz + z * fy);
        }
}

}  // namespace sxl
