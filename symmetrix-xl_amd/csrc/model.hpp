// Host-side MACE model: format-version-4 compact JSON loader and the compact
// radial tabulation.
//
// Loader semantics follow the reference's MACECPU::load_from_json
// (libsymmetrix/source/mace.cpp:2659-2959) and the format-4 H1 affine
// validation (h1_affine_schema.hpp:168-258) for the "m0_composite" and
// "pre_linear_up" bases; the radial tabulation follows CompactRadialModel
// (compact_radial.cpp:110-420).  Unsupported options (field coupling,
// pair-spline radial form, single-layer models) are rejected with an error,
// never ignored.
#pragma once

#include <string>
#include <vector>

namespace sxl {

struct RadialNetwork {
    std::vector<int> shape;
    std::vector<std::vector<double>> weights;  // [layer] row-major [out][in]
    double activation_scale = 1.0;
    bool tanh_square = false;  // output postprocess tanh(y^2) (A0/A1 density networks)
};

struct HostModel {
    int num_elements = 0;
    int channels = 0;
    int l_max = 0, L_max = 0;
    int num_lm = 0, num_LM = 0;
    double r_cut = 0.0;
    std::vector<int> atomic_numbers;
    std::vector<double> atomic_energies;
    std::string selected_head;
    std::vector<std::string> available_heads;

    // compact radial model
    double grid_min = 0.0, spline_h = 0.0;
    int spline_points = 0;
    std::vector<double> bessel_weights;
    double bessel_prefactor = 0.0;
    double cutoff_rmax = 0.0;
    int cutoff_p = 0;
    // Agnesi distance transform of the radial features (compact_radial.cpp:150-170, 238-247)
    bool agnesi = false;
    double agnesi_a = 0.0, agnesi_q = 0.0, agnesi_p = 0.0;
    std::vector<double> agnesi_radii;  // [ne] covalent radius per element type
    RadialNetwork R0, R1;
    // density normalisation: A0 /= 1 + sum_j A0net(r_ij), same for A1
    // (mace.cpp:1561-1636, 2380-2458); one-output tanh-square networks
    bool A0_scaled = false, A1_scaled = false;
    RadialNetwork A0net, A1net;

    // ZBL pair repulsion (zbl_kokkos.cpp:12-126)
    bool has_zbl = false;
    double zbl_a_exp = 0.0, zbl_a_prefactor = 0.0;
    double zbl_c[4] = {};
    std::vector<double> zbl_radii;  // indexed by atomic number
    int zbl_p = 0;

    std::vector<double> H0;   // [ne][C]
    std::vector<double> A0W;  // [ne][l_max+1][C][C]  ([in][out])

    // symmetric contraction M0: terms of all LM, grouped by LM
    std::vector<int> m0_offsets;  // [num_LM+1]
    std::vector<int> m0_degree;   // [T]
    std::vector<int> m0_index;    // [T][3]
    std::vector<double> m0_coef;  // [ne][T][C]

    std::vector<double> H1W;  // [L_max+1][C][C]

    // pre_linear_up basis (h1_affine_schema.hpp:14-24): the readout_1 and
    // H1->H2 skip maps act on x = P0^T M0_scalar (+ the residual's scalar
    // block), P = H1_product_weights; m0_composite: x = M0_scalar.
    bool pre_linear_up = false;
    std::vector<double> H1P;  // [L_max+1][C][C] ([in][out]); only l = 0 is used
    // first-interaction residual (mace.cpp:1845-1880, 2796-2825): per element
    // constants added to the pre-linear_up features; H1 gains the fused
    // residual (residual U per l), x the unfused scalar block
    bool first_residual = false;
    std::vector<double> residual;        // [ne][num_LM][C]
    std::vector<double> residual_fused;  // [ne][num_LM][C]

    std::vector<int> Phi1_l, Phi1_l1, Phi1_l2, Phi1_lme, Phi1_row;
    std::vector<double> Phi1_cg;
    std::vector<std::vector<double>> A1W;  // [l] -> [num_e[l]*C][C]

    std::vector<int> m1_degree, m1_index;  // [T1], [T1][3]
    std::vector<double> m1_coef;           // [ne][T1][C]

    std::vector<double> H2M0;  // [ne][C][C]  ([in][out]) skip map on x
    std::vector<double> H2M1;  // [C][C]
    std::vector<double> readout_q;  // [C] readout_1 on x
    int readout_hidden = 16;
    std::vector<double> readout_w1;  // [hidden][C]
    std::vector<double> readout_w2;  // [hidden]
    double readout_scale = 1.0;

    static HostModel load(const std::string& path, const std::string& head);

    // Nodal values and derivatives, [function][knot], of one radial network
    // for the unordered element pair (type_i, type_j).
    void radial_tables(const RadialNetwork& net, int type_i, int type_j,
                       std::vector<double>& values, std::vector<double>& derivs) const;

    int num_paths() const { return static_cast<int>(Phi1_l.size()); }
};

}  // namespace sxl
