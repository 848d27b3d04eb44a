// TEST INFRASTRUCTURE ONLY -- the CPU oracle for MACE energies and forces.
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
// load this code, and only as the checker (and as the timed CPU baseline).
// The product never calls it.
//
// Restatement of the reference's serial evaluator MACECPU<Precision> in its
// streamed ("generic") mode, libsymmetrix/source/mace.cpp:
//   compute_node_energies_forces order            mace.cpp:231-319
//   compute_Y (x,y,z -> z,x,y, x 2 sqrt(pi))      mace.cpp:1268-1299
//   compute_A0_streamed                           mace.cpp:1355-1403
//   compute_M0 / reverse_M0                       mace.cpp:1638-1688
//   compute_H1 / reverse_H1 (+ direct adjoint)    mace.cpp:1690-1756, 1784-1813
//   compute_Phi1_streamed                         mace.cpp:2022-2083
//   compute_A1 / reverse_A1                       mace.cpp:2304-2378
//   compute_M1 / reverse_M1                       mace.cpp:2460-2513
//   compute_H2 / reverse_H2 (format 4)            mace.cpp:2515-2619
//   pre_linear_up scalar, first-interaction residual
//                                                 mace.cpp:1759-1813, 1845-1875
//   compute_readouts                              mace.cpp:2621-2657
//   reverse_Phi1_streamed                         mace.cpp:2198-2302
//   reverse_A0_streamed                           mace.cpp:1485-1559
//   compute/reverse_A0_scaled, A1_scaled          mace.cpp:1561-1636, 2380-2458
//   ZBL pair term, in double as the device path   zbl_kokkos.cpp:76-126, 154-201
// Splines: cubic Hermite coefficients (formed in double, stored in Precision,
//   as the device path's tables, mace_kokkos_factorized_lifecycle.cpp:4002-4013)
//   and evaluation point (cubic_spline_set.cpp:32-78).
// Polynomials: evaluate_gradient_simple (multivariate_polynomial.cpp:326-355)
//   over each output's terms as the constructor stores them: a repeated
//   monomial keeps its first coefficient (multivariate_polynomial.cpp:36-46).
// Readout MLP: evaluate_gradient (multilayer_perceptron.cpp:85-160).
// Harmonics: closed-form real harmonics of the permuted unit direction; the
//   gradient is (grad P(u) - l P(u) u)/r for the degree-l homogeneous form P.
// Edges with r >= r_cut are skipped (the streamed mode's active-edge filter,
//   symmetrix/source/symmetrix/calculator.py:3088-3093).
// Node energies and directed forces are stored in double; the per-edge force
// sums are formed in Precision as in the reference loops.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

thread_local std::string g_last_error;

struct Spec {
    // dimensions
    int num_elements, channels, l_max, L_max;
    double r_cut;
    // active types for the radial cache
    int num_active;
    const int* type_to_active;  // [num_elements], -1 if inactive
    // splines: nodal values/derivatives per unordered active pair
    int spline_nodes;
    double spline_h, spline_x0;
    const double* r0_values;   // [pairs][(l_max+1)*C][nodes]
    const double* r0_derivs;
    const double* r1_values;   // [pairs][paths*C][nodes]
    const double* r1_derivs;
    // weights
    const double* H0;          // [ne][C]
    const double* A0W;         // [ne][l_max+1][C][C]
    const int* m0_offsets;     // [nLM+1] term offsets
    const int* m0_degree;      // [terms]
    const int* m0_index;       // [terms][3]
    const double* m0_coef;     // [ne][C][terms]
    const double* H1W;         // [L_max+1][C][C]
    int num_paths, num_terms;
    const int* path_l;         // [paths]
    const int* path_l1;
    const int* path_l2;
    const int* term_lme;       // [terms]
    const int* term_row;
    const double* term_cg;
    const double* const* A1W;  // [l_max+1] -> [num_e[l]*C][C]
    int m1_terms;
    const int* m1_degree;
    const int* m1_index;       // [m1_terms][3]
    const double* m1_coef;     // [ne][C][m1_terms]
    const double* H2M0;        // [ne][C][C]
    const double* H2M1;        // [C][C]
    const double* readout_q;   // [C]
    int readout_hidden;
    const double* readout_w1;  // [hidden][C]
    const double* readout_w2;  // [hidden]
    double readout_scale;
    const double* atomic_energies;  // [ne]
    const int* atomic_numbers;      // [ne]
    // ZBL
    int has_zbl;
    double zbl_a_exp, zbl_a_prefactor;
    double zbl_c[4];
    int zbl_num_radii;
    const double* zbl_radii;        // indexed by atomic number
    int zbl_p;
    // density normalisation splines: [pairs][1][nodes]
    int A0_scaled;
    const double* a0s_values;
    const double* a0s_derivs;
    int A1_scaled;
    const double* a1s_values;
    const double* a1s_derivs;
    // pre_linear_up basis: readout_1 / skip act on x = M0_scalar P0 (+ residual)
    int pre_linear_up;
    const double* H1P0;            // [C][C] ([in][out]) H1_product_weights, l = 0 block
    // first-interaction residual: H1 += fused (residual U), x += residual scalar block
    int first_residual;
    const double* residual;        // [ne][nLM][C]
    const double* residual_fused;  // [ne][nLM][C]
};

template <typename P>
P checked(double v)
{
    if (!std::isfinite(v) || std::abs(v) > static_cast<double>(std::numeric_limits<P>::max()))
        throw std::invalid_argument("model value outside the requested precision range");
    return static_cast<P>(v);
}

template <typename P>
struct SplineSet {
    P h, x0;
    int nodes, nfn;
    std::vector<P> c;  // [(4*i+q)*nfn + f]

    // Hermite coefficients formed in double from the double nodal data and
    // stored in P, as the device path builds its tables
    // (mace_kokkos_factorized_lifecycle.cpp:4002-4013); the serial CPU class
    // forms them in P (cubic_spline_set.cpp:7-29), which in FP32 loses up to
    // ~1e-4 of the value scale to cancellation at the compact grid spacing.
    void build(P h_, P x0_, int nodes_, int nfn_, const double* values, const double* derivs, double hd)
    {
        h = h_;
        x0 = x0_;
        nodes = nodes_;
        nfn = nfn_;
        c.assign(static_cast<size_t>(4) * nfn * (nodes - 1), P(0));
        for (int i = 0; i < nodes - 1; ++i)
            for (int j = 0; j < nfn; ++j) {
                const double v0 = values[static_cast<size_t>(j) * nodes + i];
                const double d0 = derivs[static_cast<size_t>(j) * nodes + i];
                const double v1 = values[static_cast<size_t>(j) * nodes + i + 1];
                const double d1 = derivs[static_cast<size_t>(j) * nodes + i + 1];
                c[(4 * i) * static_cast<size_t>(nfn) + j] = checked<P>(v0);
                c[(4 * i + 1) * static_cast<size_t>(nfn) + j] = checked<P>(d0);
                c[(4 * i + 2) * static_cast<size_t>(nfn) + j] =
                    checked<P>((-3 * v0 - 2 * hd * d0 + 3 * v1 - hd * d1) / (hd * hd));
                c[(4 * i + 3) * static_cast<size_t>(nfn) + j] =
                    checked<P>((2 * v0 + hd * d0 - 2 * v1 + hd * d1) / (hd * hd * hd));
            }
    }
    void point(P r, int& interval, P& x) const
    {
        interval = static_cast<int>(std::floor((r - x0) / h));
        x = r - x0 - h * interval;
        if (interval < 0) {
            interval = 0;
            x = 0;
        } else if (interval >= nodes - 1) {
            interval = nodes - 2;
            x = h;
        }
    }
    const P* coef(int interval) const { return c.data() + static_cast<size_t>(4) * interval * nfn; }
};

// Closed-form real harmonics (orthonormal, no Condon-Shortley phase) of the
// homogeneous polynomials in (x, y, z) = permuted unit direction, and their
// gradients with respect to the unit coordinates.
template <typename P>
void real_harmonics(int lmax, P x, P y, P z, P* v, P* gx, P* gy, P* gz)
{
    const P c00 = P(0.28209479177387814);
    const P c1 = P(0.4886025119029199);
    const P c2a = P(1.0925484305920792);
    const P c20 = P(0.31539156525252005);
    const P c22 = P(0.5462742152960396);
    const P c33 = P(0.5900435899266435);
    const P c32 = P(2.890611442640554);
    const P c31 = P(0.4570457994644658);
    const P c30 = P(0.3731763325901154);
    v[0] = c00;
    gx[0] = gy[0] = gz[0] = 0;
    if (lmax >= 1) {
        v[1] = c1 * y; gx[1] = 0; gy[1] = c1; gz[1] = 0;
        v[2] = c1 * z; gx[2] = 0; gy[2] = 0; gz[2] = c1;
        v[3] = c1 * x; gx[3] = c1; gy[3] = 0; gz[3] = 0;
    }
    if (lmax >= 2) {
        v[4] = c2a * x * y; gx[4] = c2a * y; gy[4] = c2a * x; gz[4] = 0;
        v[5] = c2a * y * z; gx[5] = 0; gy[5] = c2a * z; gz[5] = c2a * y;
        v[6] = c20 * (2 * z * z - x * x - y * y);
        gx[6] = -2 * c20 * x; gy[6] = -2 * c20 * y; gz[6] = 4 * c20 * z;
        v[7] = c2a * x * z; gx[7] = c2a * z; gy[7] = 0; gz[7] = c2a * x;
        v[8] = c22 * (x * x - y * y); gx[8] = 2 * c22 * x; gy[8] = -2 * c22 * y; gz[8] = 0;
    }
    if (lmax >= 3) {
        v[9] = c33 * y * (3 * x * x - y * y);
        gx[9] = 6 * c33 * x * y; gy[9] = c33 * (3 * x * x - 3 * y * y); gz[9] = 0;
        v[10] = c32 * x * y * z;
        gx[10] = c32 * y * z; gy[10] = c32 * x * z; gz[10] = c32 * x * y;
        v[11] = c31 * y * (4 * z * z - x * x - y * y);
        gx[11] = -2 * c31 * x * y; gy[11] = c31 * (4 * z * z - x * x - 3 * y * y);
        gz[11] = 8 * c31 * y * z;
        v[12] = c30 * z * (2 * z * z - 3 * x * x - 3 * y * y);
        gx[12] = -6 * c30 * x * z; gy[12] = -6 * c30 * y * z;
        gz[12] = c30 * (6 * z * z - 3 * x * x - 3 * y * y);
        v[13] = c31 * x * (4 * z * z - x * x - y * y);
        gx[13] = c31 * (4 * z * z - 3 * x * x - y * y); gy[13] = -2 * c31 * x * y;
        gz[13] = 8 * c31 * x * z;
        v[14] = P(0.5) * c32 * z * (x * x - y * y);
        gx[14] = c32 * x * z; gy[14] = -c32 * y * z; gz[14] = P(0.5) * c32 * (x * x - y * y);
        v[15] = c33 * x * (x * x - 3 * y * y);
        gx[15] = c33 * (3 * x * x - 3 * y * y); gy[15] = -6 * c33 * x * y; gz[15] = 0;
    }
}

// ZBL pair term of atomic numbers (Zu, Zv) at distance r: value and d/dr of
// 0.5 V(r) envelope(r), in double (zbl_kokkos.cpp:37-52, 76-126).
void zbl_pair_term(double a_exp, double a_prefactor, const double* c, const double* radii, int num_radii, int p,
                   int Zu, int Zv, double r, double& value, double& gradient)
{
    if (Zu < 0 || Zv < 0 || Zu >= num_radii || Zv >= num_radii)
        throw std::out_of_range("ZBL covalent radius index out of range");
    const double denominator = std::pow(static_cast<double>(Zu), a_exp) + std::pow(static_cast<double>(Zv), a_exp);
    const double inverse_a = denominator / (a_prefactor * 0.529);
    const double prefactor = 14.3996 * static_cast<double>(Zu * Zv);
    const double r_max = radii[Zu] + radii[Zv];
    if (r >= r_max) {
        value = gradient = 0.0;
        return;
    }
    const double r_over_a = r * inverse_a;
    const double e0 = c[0] * std::exp(-3.2 * r_over_a);
    const double e1 = c[1] * std::exp(-0.9423 * r_over_a);
    const double e2 = c[2] * std::exp(-0.4028 * r_over_a);
    const double e3 = c[3] * std::exp(-0.2016 * r_over_a);
    const double phi = e0 + e1 + e2 + e3;
    const double dphi = inverse_a * (-3.2 * e0 - 0.9423 * e1 - 0.4028 * e2 - 0.2016 * e3);
    const double inverse_r = 1.0 / r;
    const double bare = prefactor * inverse_r * phi;
    const double bare_gradient = prefactor * inverse_r * inverse_r * (r * dphi - phi);
    const double k0 = (p + 1.0) * (p + 2.0) / 2.0, k1 = p * (p + 2.0), k2 = p * (p + 1.0) / 2.0;
    const double x = r / r_max;
    const double xpm1 = std::pow(x, p - 1), xp = xpm1 * x, xp1 = xp * x, xp2 = xp1 * x;
    const double envelope = 1.0 - k0 * xp + k1 * xp1 - k2 * xp2;
    const double envelope_gradient = (-k0 * p * xpm1 + k1 * (p + 1.0) * xp - k2 * (p + 2.0) * xp1) / r_max;
    value = 0.5 * bare * envelope;
    gradient = 0.5 * (bare * envelope_gradient + bare_gradient * envelope);
}

template <typename P>
struct Oracle {
    int ne, C, lmax, Lmax, nlm, nLM, num_active;
    double r_cut;
    std::vector<int> type_to_active;
    std::vector<SplineSet<P>> spl0, spl1;
    std::vector<P> H0, A0W, H1W, H2M0, H2M1, q, W1, W2;
    bool pre_linear_up = false, first_residual = false;
    std::vector<P> P0, residual, residual_fused;
    int hidden;
    P scale;
    std::vector<double> E0;
    std::vector<int> m0_off, m0_deg, m0_idx;
    std::vector<char> m0_used, m1_used;  // first occurrence of each monomial per output
    std::vector<P> m0_coef;
    int m0_terms;
    std::vector<int> m1_deg, m1_idx;
    std::vector<P> m1_coef;
    int m1_terms;
    int num_paths, num_terms, num_rows, num_lme;
    std::vector<int> path_l, path_l1, path_l2, path_row0, term_lme, term_row, num_e;
    std::vector<P> term_cg;
    std::vector<std::vector<P>> A1W;
    std::vector<int> Z;
    bool has_zbl = false;
    double zbl_a_exp = 0, zbl_a_prefactor = 0, zbl_c[4] = {};
    std::vector<double> zbl_radii;
    int zbl_p = 0;
    bool A0_scaled = false, A1_scaled = false;
    std::vector<SplineSet<P>> splA0, splA1;

    explicit Oracle(const Spec& s)
    {
        ne = s.num_elements;
        C = s.channels;
        lmax = s.l_max;
        Lmax = s.L_max;
        if (lmax < 0 || lmax > 3 || Lmax < 0 || Lmax > lmax)
            throw std::invalid_argument("oracle supports l_max <= 3 and L_max <= l_max");
        nlm = (lmax + 1) * (lmax + 1);
        nLM = (Lmax + 1) * (Lmax + 1);
        r_cut = s.r_cut;
        num_active = s.num_active;
        type_to_active.assign(s.type_to_active, s.type_to_active + ne);
        const int pairs = num_active * (num_active + 1) / 2;
        num_paths = s.num_paths;
        const size_t n0 = static_cast<size_t>(lmax + 1) * C;
        const size_t n1 = static_cast<size_t>(num_paths) * C;
        spl0.resize(pairs);
        spl1.resize(pairs);
        const P h = checked<P>(s.spline_h), x0 = checked<P>(s.spline_x0);
        for (int p = 0; p < pairs; ++p) {
            spl0[p].build(h, x0, s.spline_nodes, static_cast<int>(n0),
                          s.r0_values + p * n0 * s.spline_nodes, s.r0_derivs + p * n0 * s.spline_nodes, s.spline_h);
            spl1[p].build(h, x0, s.spline_nodes, static_cast<int>(n1),
                          s.r1_values + p * n1 * s.spline_nodes, s.r1_derivs + p * n1 * s.spline_nodes, s.spline_h);
        }
        auto conv = [](const double* src, size_t n) {
            std::vector<P> out(n);
            for (size_t i = 0; i < n; ++i) out[i] = checked<P>(src[i]);
            return out;
        };
        H0 = conv(s.H0, static_cast<size_t>(ne) * C);
        A0W = conv(s.A0W, static_cast<size_t>(ne) * (lmax + 1) * C * C);
        H1W = conv(s.H1W, static_cast<size_t>(Lmax + 1) * C * C);
        m0_off.assign(s.m0_offsets, s.m0_offsets + nLM + 1);
        m0_terms = m0_off[nLM];
        m0_deg.assign(s.m0_degree, s.m0_degree + m0_terms);
        m0_idx.assign(s.m0_index, s.m0_index + 3 * m0_terms);
        m0_used.assign(m0_terms, 1);
        for (int LM = 0; LM < nLM; ++LM)
            first_terms(m0_deg.data(), m0_idx.data(), m0_off[LM], m0_off[LM + 1], m0_used.data());
        m0_coef = conv(s.m0_coef, static_cast<size_t>(ne) * C * m0_terms);
        num_terms = s.num_terms;
        path_l.assign(s.path_l, s.path_l + num_paths);
        path_l1.assign(s.path_l1, s.path_l1 + num_paths);
        path_l2.assign(s.path_l2, s.path_l2 + num_paths);
        term_lme.assign(s.term_lme, s.term_lme + num_terms);
        term_row.assign(s.term_row, s.term_row + num_terms);
        term_cg = conv(s.term_cg, num_terms);
        num_e.assign(lmax + 1, 0);
        num_lme = 0;
        num_rows = 0;
        for (int p = 0; p < num_paths; ++p) {
            num_e[path_l[p]] += 1;
            num_lme += 2 * path_l[p] + 1;
            path_row0.push_back(num_rows);
            num_rows += (2 * path_l1[p] + 1) * (2 * path_l2[p] + 1);
        }
        A1W.resize(lmax + 1);
        for (int l = 0; l <= lmax; ++l)
            A1W[l] = conv(s.A1W[l], static_cast<size_t>(num_e[l]) * C * C);
        m1_terms = s.m1_terms;
        m1_deg.assign(s.m1_degree, s.m1_degree + m1_terms);
        m1_idx.assign(s.m1_index, s.m1_index + 3 * m1_terms);
        m1_used.assign(m1_terms, 1);
        first_terms(m1_deg.data(), m1_idx.data(), 0, m1_terms, m1_used.data());
        m1_coef = conv(s.m1_coef, static_cast<size_t>(ne) * C * m1_terms);
        H2M0 = conv(s.H2M0, static_cast<size_t>(ne) * C * C);
        H2M1 = conv(s.H2M1, static_cast<size_t>(C) * C);
        q = conv(s.readout_q, C);
        pre_linear_up = s.pre_linear_up != 0;
        if (pre_linear_up) P0 = conv(s.H1P0, static_cast<size_t>(C) * C);
        first_residual = s.first_residual != 0;
        if (first_residual) {
            residual = conv(s.residual, static_cast<size_t>(ne) * nLM * C);
            residual_fused = conv(s.residual_fused, static_cast<size_t>(ne) * nLM * C);
        }
        hidden = s.readout_hidden;
        W1 = conv(s.readout_w1, static_cast<size_t>(hidden) * C);
        W2 = conv(s.readout_w2, hidden);
        scale = checked<P>(s.readout_scale);
        E0.assign(s.atomic_energies, s.atomic_energies + ne);
        Z.assign(s.atomic_numbers, s.atomic_numbers + ne);
        has_zbl = s.has_zbl != 0;
        if (has_zbl) {
            zbl_a_exp = s.zbl_a_exp;
            zbl_a_prefactor = s.zbl_a_prefactor;
            for (int q = 0; q < 4; ++q) zbl_c[q] = s.zbl_c[q];
            zbl_radii.assign(s.zbl_radii, s.zbl_radii + s.zbl_num_radii);
            zbl_p = s.zbl_p;
        }
        A0_scaled = s.A0_scaled != 0;
        A1_scaled = s.A1_scaled != 0;
        if (A0_scaled) {
            splA0.resize(pairs);
            for (int p = 0; p < pairs; ++p)
                splA0[p].build(h, x0, s.spline_nodes, 1, s.a0s_values + static_cast<size_t>(p) * s.spline_nodes,
                               s.a0s_derivs + static_cast<size_t>(p) * s.spline_nodes, s.spline_h);
        }
        if (A1_scaled) {
            splA1.resize(pairs);
            for (int p = 0; p < pairs; ++p)
                splA1[p].build(h, x0, s.spline_nodes, 1, s.a1s_values + static_cast<size_t>(p) * s.spline_nodes,
                               s.a1s_derivs + static_cast<size_t>(p) * s.spline_nodes, s.spline_h);
        }
    }

    void zbl_pair(int Zu, int Zv, double r, double& value, double& gradient) const
    {
        zbl_pair_term(zbl_a_exp, zbl_a_prefactor, zbl_c, zbl_radii.data(), static_cast<int>(zbl_radii.size()),
                      zbl_p, Zu, Zv, r, value, gradient);
    }

    // 1 + sum over the receiver's neighbours of a density spline
    // (compute_A0_scaled / compute_A1_scaled, mace.cpp:1573-1580)
    P scale_factor(const std::vector<SplineSet<P>>& spl, int i, const long long* first, const int* types,
                   const int* neigh_types, const double* r) const
    {
        P s = 1.0;
        for (long long e = first[i]; e < first[i + 1]; ++e) {
            const auto& sp = spl[pair_index(types[i], neigh_types[e])];
            int iv;
            P x;
            sp.point(static_cast<P>(r[e]), iv, x);
            const P* c = sp.coef(iv);
            s += c[0] + c[1] * x + c[2] * (x * x) + c[3] * (x * x * x);
        }
        return s;
    }

    // reverse_A0_scaled / reverse_A1_scaled (mace.cpp:1584-1636, 2404-2458):
    // forces += (adj . feat) / s * f'(r) r_hat for every neighbour, adj /= s.
    void reverse_scale(const std::vector<SplineSet<P>>& spl, int N, const long long* first, const int* types,
                       const int* neigh_types, const double* xyz, const double* r, const P* feat, P* adj,
                       double* forces) const
    {
        const size_t width = static_cast<size_t>(nlm) * C;
#pragma omp parallel for schedule(static)
        for (int i = 0; i < N; ++i) {
            const P s = scale_factor(spl, i, first, types, neigh_types, r);
            P dot = 0;
            const P* f = feat + i * width;
            P* a = adj + i * width;
            for (size_t lmk = 0; lmk < width; ++lmk) dot += a[lmk] * f[lmk];
            for (long long e = first[i]; e < first[i + 1]; ++e) {
                const auto& sp = spl[pair_index(types[i], neigh_types[e])];
                int iv;
                P x;
                sp.point(static_cast<P>(r[e]), iv, x);
                const P* c = sp.coef(iv);
                const P d = static_cast<P>(c[1] + 2.0 * c[2] * x + 3.0 * c[3] * x * x);
                const P force_scale = dot / s * d;
                for (int q = 0; q < 3; ++q)
                    forces[3 * e + q] += static_cast<double>(force_scale * static_cast<P>(xyz[3 * e + q] / r[e]));
            }
            for (size_t lmk = 0; lmk < width; ++lmk) a[lmk] /= s;
        }
    }

    int pair_index(int ti, int tj) const
    {
        const int ai = type_to_active.at(ti), aj = type_to_active.at(tj);
        if (ai < 0 || aj < 0) throw std::runtime_error("radial cache is not prepared for an active type");
        const int n = num_active;
        return ai <= aj ? ai * (2 * n - ai - 1) / 2 + aj : aj * (2 * n - aj - 1) / 2 + ai;
    }

    // Terms of one polynomial output that the reference keeps: it stores the
    // (monomial, coefficient) pairs in a std::map keyed by the exact index
    // vector, and map::insert ignores a key already present, so a monomial
    // listed again keeps its first coefficient; [0,1] and [1,0] are distinct
    // keys (multivariate_polynomial.cpp:36-46).  used[t] = 0 marks a repeat.
    static void first_terms(const int* deg, const int* idx, int begin, int end, char* used)
    {
        for (int t = begin; t < end; ++t) {
            used[t] = 1;
            for (int u = begin; u < t && used[t]; ++u)
                if (used[u] && deg[u] == deg[t] && std::equal(idx + 3 * u, idx + 3 * u + deg[t], idx + 3 * t))
                    used[t] = 0;
        }
    }

    // polynomial value and gradient (evaluate_gradient_simple) over the terms
    // with used[t] != 0
    static P poly(const P* coef, const int* deg, const int* idx, const char* used, int begin, int end, const P* x,
                  P* g, int nvar)
    {
        P f = 0;
        for (int v = 0; v < nvar; ++v) g[v] = 0;
        for (int t = begin; t < end; ++t) {
            if (!used[t]) continue;
            const int* i = idx + 3 * t;
            const P c = coef[t];
            if (deg[t] == 1) {
                f += c * x[i[0]];
                g[i[0]] += c;
            } else if (deg[t] == 2) {
                f += c * x[i[0]] * x[i[1]];
                g[i[0]] += c * x[i[1]];
                g[i[1]] += c * x[i[0]];
            } else {
                f += c * x[i[0]] * x[i[1]] * x[i[2]];
                g[i[0]] += c * x[i[1]] * x[i[2]];
                g[i[1]] += c * x[i[0]] * x[i[2]];
                g[i[2]] += c * x[i[0]] * x[i[1]];
            }
        }
        return f;
    }

    void compute(int N, const int* types, const int* num_neigh, const int* neigh_idx,
                 const int* neigh_types, const double* xyz, const double* r, double* energies,
                 double* forces, int num_threads)
    {
#ifdef _OPENMP
        if (num_threads > 0) omp_set_num_threads(num_threads);
#endif
        std::vector<long long> first(N + 1, 0);
        for (int i = 0; i < N; ++i) first[i + 1] = first[i] + num_neigh[i];
        const long long E = first[N];
        const P rc = static_cast<P>(r_cut);
        for (long long e = 0; e < 3 * E; ++e) forces[e] = 0.0;
        for (int i = 0; i < N; ++i) energies[i] = 0.0;

        // ---- ZBL (every neighbour, double) ----
        if (has_zbl) {
#pragma omp parallel for schedule(static)
            for (int i = 0; i < N; ++i) {
                double e_i = 0.0;
                for (long long e = first[i]; e < first[i + 1]; ++e) {
                    double v, g;
                    zbl_pair(Z.at(types[i]), Z.at(neigh_types[e]), r[e], v, g);
                    e_i += v;
                    for (int q = 0; q < 3; ++q) forces[3 * e + q] -= xyz[3 * e + q] / r[e] * g;
                }
                energies[i] += e_i;
            }
        }

        // ---- compute_Y: values and gradients w.r.t. xyz (unshuffled) ----
        std::vector<P> Y(static_cast<size_t>(E) * nlm), Yg(static_cast<size_t>(E) * 3 * nlm);
#pragma omp parallel for schedule(static)
        for (long long e = 0; e < E; ++e) {
            const P ex = static_cast<P>(xyz[3 * e]), ey = static_cast<P>(xyz[3 * e + 1]),
                    ez = static_cast<P>(xyz[3 * e + 2]);
            const P rr = std::sqrt(ex * ex + ey * ey + ez * ez);
            P v[16], gx[16], gy[16], gz[16];
            P* Ye = Y.data() + e * nlm;
            P* Ge = Yg.data() + e * 3 * nlm;
            if (rr == P(0)) {
                for (int lm = 0; lm < nlm; ++lm) {
                    Ye[lm] = lm == 0 ? P(1) : P(0);
                    Ge[lm] = Ge[nlm + lm] = Ge[2 * nlm + lm] = 0;
                }
                continue;
            }
            // permuted unit direction (z, x, y)
            const P u0 = ez / rr, u1 = ex / rr, u2 = ey / rr;
            real_harmonics<P>(lmax, u0, u1, u2, v, gx, gy, gz);
            const P norm = P(3.5449077018110318);
            for (int l = 0; l <= lmax; ++l)
                for (int lm = l * l; lm < (l + 1) * (l + 1); ++lm) {
                    // d/du of P(u/|u|) = grad P - l P u, then / r
                    const P d0 = (gx[lm] - l * v[lm] * u0) / rr;
                    const P d1 = (gy[lm] - l * v[lm] * u1) / rr;
                    const P d2 = (gz[lm] - l * v[lm] * u2) / rr;
                    Ye[lm] = norm * v[lm];
                    // unshuffle: d/dx = d/du1, d/dy = d/du2, d/dz = d/du0
                    Ge[lm] = norm * d1;
                    Ge[nlm + lm] = norm * d2;
                    Ge[2 * nlm + lm] = norm * d0;
                }
        }

        // ---- compute_A0_streamed ----
        std::vector<P> A0(static_cast<size_t>(N) * nlm * C);
#pragma omp parallel
        {
            std::vector<P> Phi0(static_cast<size_t>(nlm) * C), rad(C);
#pragma omp for schedule(dynamic, 16)
            for (int i = 0; i < N; ++i) {
                std::fill(Phi0.begin(), Phi0.end(), P(0));
                for (long long e = first[i]; e < first[i + 1]; ++e) {
                    if (!(static_cast<P>(r[e]) < rc)) continue;
                    const auto& sp = spl0[pair_index(types[i], neigh_types[e])];
                    int iv;
                    P x;
                    sp.point(static_cast<P>(r[e]), iv, x);
                    const P* c = sp.coef(iv);
                    const P xx = x * x, xxx = xx * x;
                    const P* Ye = Y.data() + e * nlm;
                    const P* h0 = H0.data() + static_cast<size_t>(neigh_types[e]) * C;
                    for (int l = 0; l <= lmax; ++l) {
                        for (int k = 0; k < C; ++k) {
                            const int f = l * C + k;
                            rad[k] = c[f] + c[sp.nfn + f] * x + c[2 * sp.nfn + f] * xx +
                                     c[3 * sp.nfn + f] * xxx;
                        }
                        for (int lm = l * l; lm < (l + 1) * (l + 1); ++lm) {
                            P* ph = Phi0.data() + static_cast<size_t>(lm) * C;
                            const P y = Ye[lm];
                            for (int k = 0; k < C; ++k) ph[k] += rad[k] * y * h0[k];
                        }
                    }
                }
                for (int l = 0; l <= lmax; ++l) {
                    const P* W = A0W.data() + (static_cast<size_t>(types[i]) * (lmax + 1) + l) * C * C;
                    for (int lm = l * l; lm < (l + 1) * (l + 1); ++lm) {
                        P* out = A0.data() + (static_cast<size_t>(i) * nlm + lm) * C;
                        const P* ph = Phi0.data() + static_cast<size_t>(lm) * C;
                        for (int ko = 0; ko < C; ++ko) out[ko] = 0;
                        for (int ki = 0; ki < C; ++ki) {
                            const P a = ph[ki];
                            const P* w = W + static_cast<size_t>(ki) * C;
                            for (int ko = 0; ko < C; ++ko) out[ko] += a * w[ko];
                        }
                    }
                }
            }
        }

        // ---- compute_A0_scaled ----
        if (A0_scaled) {
#pragma omp parallel for schedule(static)
            for (int i = 0; i < N; ++i) {
                const P sf = scale_factor(splA0, i, first.data(), types, neigh_types, r);
                P* a = A0.data() + static_cast<size_t>(i) * nlm * C;
                for (size_t lmk = 0; lmk < static_cast<size_t>(nlm) * C; ++lmk) a[lmk] /= sf;
            }
        }

        // ---- compute_M0 (gradient kept) ----
        std::vector<P> M0(static_cast<size_t>(N) * nLM * C),
            M0g(static_cast<size_t>(N) * nLM * nlm * C);
#pragma omp parallel for schedule(static)
        for (int i = 0; i < N; ++i) {
            P x[16], g[16];
            for (int k = 0; k < C; ++k) {
                for (int lm = 0; lm < nlm; ++lm) x[lm] = A0[(static_cast<size_t>(i) * nlm + lm) * C + k];
                const P* coef = m0_coef.data() + (static_cast<size_t>(types[i]) * C + k) * m0_terms;
                for (int LM = 0; LM < nLM; ++LM) {
                    const P f = poly(coef, m0_deg.data(), m0_idx.data(), m0_used.data(), m0_off[LM], m0_off[LM + 1],
                                     x, g, nlm);
                    M0[(static_cast<size_t>(i) * nLM + LM) * C + k] = f;
                    for (int lm = 0; lm < nlm; ++lm)
                        M0g[((static_cast<size_t>(i) * nLM + LM) * nlm + lm) * C + k] = g[lm];
                }
            }
        }

        // ---- compute_H1, capture_h1_affine_scalar, add_H1_first_residual
        // (mace.cpp:1690-1783, 1845-1875): H1 = M0 H1_W (+ fused residual of
        // the node's element); readout input x = M0 scalar block
        // (m0_composite) or M0_scalar P0 (+ residual scalar block) ----
        std::vector<P> H1(static_cast<size_t>(N) * nLM * C);
        gemm_blocks(N, nLM, Lmax, M0.data(), H1W.data(), H1.data(), false);
        if (first_residual)
            for (int i = 0; i < N; ++i) {
                const P* res = residual_fused.data() + static_cast<size_t>(types[i]) * nLM * C;
                P* h = H1.data() + static_cast<size_t>(i) * nLM * C;
                for (int j = 0; j < nLM * C; ++j) h[j] += res[j];
            }
        std::vector<P> xs_pre;
        if (pre_linear_up) {
            xs_pre.assign(static_cast<size_t>(N) * C, P(0));
            for (int i = 0; i < N; ++i) {
                const P* m0 = M0.data() + static_cast<size_t>(i) * nLM * C;
                P* x = xs_pre.data() + static_cast<size_t>(i) * C;
                for (int k = 0; k < C; ++k) {
                    P acc = 0;
                    for (int kp = 0; kp < C; ++kp) acc += m0[kp] * P0[static_cast<size_t>(kp) * C + k];
                    x[k] = acc;
                }
                if (first_residual) {
                    const P* res = residual.data() + static_cast<size_t>(types[i]) * nLM * C;
                    for (int k = 0; k < C; ++k) x[k] += res[k];
                }
            }
        }

        // ---- compute_Phi1_streamed ----
        std::vector<P> Phi1(static_cast<size_t>(N) * num_lme * C);
#pragma omp parallel
        {
            std::vector<P> Phi1r(static_cast<size_t>(num_rows) * C), rad(C);
#pragma omp for schedule(dynamic, 16)
            for (int i = 0; i < N; ++i) {
                std::fill(Phi1r.begin(), Phi1r.end(), P(0));
                for (long long e = first[i]; e < first[i + 1]; ++e) {
                    if (!(static_cast<P>(r[e]) < rc)) continue;
                    const auto& sp = spl1[pair_index(types[i], neigh_types[e])];
                    int iv;
                    P x;
                    sp.point(static_cast<P>(r[e]), iv, x);
                    const P* c = sp.coef(iv);
                    const P xx = x * x, xxx = xx * x;
                    const P* Ye = Y.data() + e * nlm;
                    const P* Hs = H1.data() + static_cast<size_t>(neigh_idx[e]) * nLM * C;
                    int row = 0;
                    for (int p = 0; p < num_paths; ++p) {
                        for (int k = 0; k < C; ++k) {
                            const int f = p * C + k;
                            rad[k] = c[f] + c[sp.nfn + f] * x + c[2 * sp.nfn + f] * xx +
                                     c[3 * sp.nfn + f] * xxx;
                        }
                        const int l1 = path_l1[p], l2 = path_l2[p];
                        for (int lm1 = l1 * l1; lm1 <= l1 * (l1 + 2); ++lm1) {
                            const P y = Ye[lm1];
                            for (int lm2 = l2 * l2; lm2 <= l2 * (l2 + 2); ++lm2) {
                                const P* h = Hs + static_cast<size_t>(lm2) * C;
                                P* out = Phi1r.data() + static_cast<size_t>(row) * C;
                                for (int k = 0; k < C; ++k) out[k] += rad[k] * y * h[k];
                                ++row;
                            }
                        }
                    }
                }
                P* out = Phi1.data() + static_cast<size_t>(i) * num_lme * C;
                std::fill(out, out + static_cast<size_t>(num_lme) * C, P(0));
                for (int t = 0; t < num_terms; ++t) {
                    P* o = out + static_cast<size_t>(term_lme[t]) * C;
                    const P* src = Phi1r.data() + static_cast<size_t>(term_row[t]) * C;
                    const P cg = term_cg[t];
                    for (int k = 0; k < C; ++k) o[k] += cg * src[k];
                }
            }
        }

        // ---- compute_A1 ----
        std::vector<P> A1(static_cast<size_t>(N) * nlm * C, P(0));
#pragma omp parallel for schedule(static)
        for (int i = 0; i < N; ++i) {
            const P* ph = Phi1.data() + static_cast<size_t>(i) * num_lme * C;
            P* a1 = A1.data() + static_cast<size_t>(i) * nlm * C;
            for (int l = 0; l <= lmax; ++l) {
                const int K = num_e[l] * C;
                for (int m = 0; m < 2 * l + 1; ++m) {
                    P* out = a1 + static_cast<size_t>(m) * C;
                    const P* in = ph + static_cast<size_t>(m) * K;
                    for (int kk = 0; kk < K; ++kk) {
                        const P a = in[kk];
                        const P* w = A1W[l].data() + static_cast<size_t>(kk) * C;
                        for (int ko = 0; ko < C; ++ko) out[ko] += a * w[ko];
                    }
                }
                ph += static_cast<size_t>(2 * l + 1) * K;
                a1 += static_cast<size_t>(2 * l + 1) * C;
            }
        }

        // ---- compute_A1_scaled ----
        if (A1_scaled) {
#pragma omp parallel for schedule(static)
            for (int i = 0; i < N; ++i) {
                const P sf = scale_factor(splA1, i, first.data(), types, neigh_types, r);
                P* a = A1.data() + static_cast<size_t>(i) * nlm * C;
                for (size_t lmk = 0; lmk < static_cast<size_t>(nlm) * C; ++lmk) a[lmk] /= sf;
            }
        }

        // ---- compute_M1, compute_H2, compute_readouts, reverse_H2, reverse_M1 ----
        std::vector<P> direct(static_cast<size_t>(N) * C), A1adj(static_cast<size_t>(N) * nlm * C);
#pragma omp parallel
        {
            std::vector<P> M1(C), M1g(static_cast<size_t>(nlm) * C), H2(C), H2adj(C), hid(hidden),
                dact(hidden), M1adj(C);
#pragma omp for schedule(static)
            for (int i = 0; i < N; ++i) {
                const int ti = types[i];
                P x[16], g[16];
                for (int k = 0; k < C; ++k) {
                    for (int lm = 0; lm < nlm; ++lm) x[lm] = A1[(static_cast<size_t>(i) * nlm + lm) * C + k];
                    const P* coef = m1_coef.data() + (static_cast<size_t>(ti) * C + k) * m1_terms;
                    M1[k] = poly(coef, m1_deg.data(), m1_idx.data(), m1_used.data(), 0, m1_terms, x, g, nlm);
                    for (int lm = 0; lm < nlm; ++lm) M1g[static_cast<size_t>(lm) * C + k] = g[lm];
                }
                const P* xs = pre_linear_up ? xs_pre.data() + static_cast<size_t>(i) * C
                                            : M0.data() + static_cast<size_t>(i) * nLM * C;  // scalar block
                const P* T = H2M0.data() + static_cast<size_t>(ti) * C * C;
                for (int o = 0; o < C; ++o) {
                    P acc = 0;
                    for (int in = 0; in < C; ++in) acc += T[static_cast<size_t>(in) * C + o] * xs[in];
                    for (int in = 0; in < C; ++in) acc += H2M1[static_cast<size_t>(in) * C + o] * M1[in];
                    H2[o] = acc;
                }
                double energy = E0[ti];
                P e1 = 0;
                for (int k = 0; k < C; ++k) e1 += q[k] * xs[k];
                energy += e1;
                // readout_2: [C, hidden, 1], SiLU x scale on the hidden layer
                P out = 0;
                for (int h = 0; h < hidden; ++h) {
                    P z = 0;
                    for (int k = 0; k < C; ++k) z += W1[static_cast<size_t>(h) * C + k] * H2[k];
                    const P sig = P(1) / (P(1) + std::exp(-z));
                    hid[h] = scale * z * sig;
                    dact[h] = scale * sig + scale * z * sig * (1 - sig);
                    out += W2[h] * hid[h];
                }
                energy += out;
                energies[i] += energy;
                for (int k = 0; k < C; ++k) {
                    P g2 = 0;
                    for (int h = 0; h < hidden; ++h) g2 += W2[h] * dact[h] * W1[static_cast<size_t>(h) * C + k];
                    H2adj[k] = g2;
                }
                // reverse_H2 (v4): direct = q + T_z H2_adj ; M1_adj = W H2_adj
                P* dir = direct.data() + static_cast<size_t>(i) * C;
                for (int in = 0; in < C; ++in) {
                    P acc = q[in], acc1 = 0;
                    for (int o = 0; o < C; ++o) {
                        acc += T[static_cast<size_t>(in) * C + o] * H2adj[o];
                        acc1 += H2M1[static_cast<size_t>(in) * C + o] * H2adj[o];
                    }
                    dir[in] = acc;
                    M1adj[in] = acc1;
                }
                // reverse_M1
                for (int lm = 0; lm < nlm; ++lm)
                    for (int k = 0; k < C; ++k)
                        A1adj[(static_cast<size_t>(i) * nlm + lm) * C + k] =
                            M1g[static_cast<size_t>(lm) * C + k] * M1adj[k];
            }
        }

        // ---- reverse_A1_scaled ----
        if (A1_scaled)
            reverse_scale(splA1, N, first.data(), types, neigh_types, xyz, r, A1.data(), A1adj.data(), forces);

        // ---- reverse_A1: dPhi1 = A1_adj W^T ----
        std::vector<P> dPhi1(static_cast<size_t>(N) * num_lme * C);
#pragma omp parallel for schedule(static)
        for (int i = 0; i < N; ++i) {
            const P* a = A1adj.data() + static_cast<size_t>(i) * nlm * C;
            P* d = dPhi1.data() + static_cast<size_t>(i) * num_lme * C;
            for (int l = 0; l <= lmax; ++l) {
                const int K = num_e[l] * C;
                for (int m = 0; m < 2 * l + 1; ++m) {
                    const P* in = a + static_cast<size_t>(m) * C;
                    P* out = d + static_cast<size_t>(m) * K;
                    for (int kk = 0; kk < K; ++kk) {
                        const P* w = A1W[l].data() + static_cast<size_t>(kk) * C;
                        P acc = 0;
                        for (int ko = 0; ko < C; ++ko) acc += in[ko] * w[ko];
                        out[kk] = acc;
                    }
                }
                a += static_cast<size_t>(2 * l + 1) * C;
                d += static_cast<size_t>(2 * l + 1) * K;
            }
        }

        // ---- reverse_Phi1_streamed: forces and H1_adj (source scatter) ----
        const int threads =
#ifdef _OPENMP
            omp_get_max_threads();
#else
            1;
#endif
        std::vector<std::vector<P>> H1adj_t(threads);
#pragma omp parallel
        {
            int tid = 0;
#ifdef _OPENMP
            tid = omp_get_thread_num();
#endif
            auto& H1adj = H1adj_t[tid];
            H1adj.assign(static_cast<size_t>(N) * nLM * C, P(0));
            std::vector<P> dPhi1r(static_cast<size_t>(num_rows) * C), rad(C), drad(C);
#pragma omp for schedule(dynamic, 16)
            for (int i = 0; i < N; ++i) {
                std::fill(dPhi1r.begin(), dPhi1r.end(), P(0));
                const P* dP = dPhi1.data() + static_cast<size_t>(i) * num_lme * C;
                for (int t = 0; t < num_terms; ++t) {
                    P* o = dPhi1r.data() + static_cast<size_t>(term_row[t]) * C;
                    const P* src = dP + static_cast<size_t>(term_lme[t]) * C;
                    const P cg = term_cg[t];
                    for (int k = 0; k < C; ++k) o[k] += cg * src[k];
                }
                for (long long e = first[i]; e < first[i + 1]; ++e) {
                    if (!(static_cast<P>(r[e]) < rc)) continue;
                    const auto& sp = spl1[pair_index(types[i], neigh_types[e])];
                    int iv;
                    P x;
                    sp.point(static_cast<P>(r[e]), iv, x);
                    const P* c = sp.coef(iv);
                    const P xx = x * x, xxx = xx * x;
                    const P dx = static_cast<P>(xyz[3 * e] / r[e]);
                    const P dy = static_cast<P>(xyz[3 * e + 1] / r[e]);
                    const P dz = static_cast<P>(xyz[3 * e + 2] / r[e]);
                    const P* Ye = Y.data() + e * nlm;
                    const P* Ge = Yg.data() + e * 3 * nlm;
                    const P* Hs = H1.data() + static_cast<size_t>(neigh_idx[e]) * nLM * C;
                    P* Ha = H1adj.data() + static_cast<size_t>(neigh_idx[e]) * nLM * C;
                    P fx = 0, fy = 0, fz = 0;
                    int row = 0;
                    for (int p = 0; p < num_paths; ++p) {
                        for (int k = 0; k < C; ++k) {
                            const int f = p * C + k;
                            rad[k] = c[f] + c[sp.nfn + f] * x + c[2 * sp.nfn + f] * xx +
                                     c[3 * sp.nfn + f] * xxx;
                            // the reference forms the derivative with double literals
                            // (cubic_spline_set.cpp:71-73), i.e. in double
                            drad[k] = static_cast<P>(c[sp.nfn + f] + 2.0 * c[2 * sp.nfn + f] * x +
                                                     3.0 * c[3 * sp.nfn + f] * xx);
                        }
                        const int l1 = path_l1[p], l2 = path_l2[p];
                        for (int lm1 = l1 * l1; lm1 <= l1 * (l1 + 2); ++lm1) {
                            const P y = Ye[lm1];
                            const P gx = Ge[lm1], gy = Ge[nlm + lm1], gz = Ge[2 * nlm + lm1];
                            for (int lm2 = l2 * l2; lm2 <= l2 * (l2 + 2); ++lm2) {
                                const P* h = Hs + static_cast<size_t>(lm2) * C;
                                P* ha = Ha + static_cast<size_t>(lm2) * C;
                                const P* adj = dPhi1r.data() + static_cast<size_t>(row) * C;
                                for (int k = 0; k < C; ++k) {
                                    const P a = adj[k];
                                    const P s = h[k];
                                    const P radial_force = drad[k] * y * s;
                                    const P angular_force = rad[k] * s;
                                    fx -= a * (dx * radial_force + angular_force * gx);
                                    fy -= a * (dy * radial_force + angular_force * gy);
                                    fz -= a * (dz * radial_force + angular_force * gz);
                                    ha[k] += rad[k] * y * a;
                                }
                                ++row;
                            }
                        }
                    }
                    forces[3 * e] += fx;
                    forces[3 * e + 1] += fy;
                    forces[3 * e + 2] += fz;
                }
            }
        }
        std::vector<P> H1adj(static_cast<size_t>(N) * nLM * C, P(0));
        for (int t = 0; t < threads; ++t)
            if (!H1adj_t[t].empty())
                for (size_t j = 0; j < H1adj.size(); ++j) H1adj[j] += H1adj_t[t][j];
        H1adj_t.clear();

        // ---- reverse_H1 + direct adjoint ----
        std::vector<P> M0adj(static_cast<size_t>(N) * nLM * C);
        gemm_blocks(N, nLM, Lmax, H1adj.data(), H1W.data(), M0adj.data(), true);
        // add_h1_affine_direct_adjoint (mace.cpp:1784-1813): M0_adj scalar
        // block += direct (m0_composite) or P0 direct (pre_linear_up)
        for (int i = 0; i < N; ++i) {
            const P* dir = direct.data() + static_cast<size_t>(i) * C;
            P* adj = M0adj.data() + static_cast<size_t>(i) * nLM * C;
            if (pre_linear_up) {
                for (int kp = 0; kp < C; ++kp) {
                    P acc = 0;
                    for (int k = 0; k < C; ++k) acc += P0[static_cast<size_t>(kp) * C + k] * dir[k];
                    adj[kp] += acc;
                }
            } else {
                for (int k = 0; k < C; ++k) adj[k] += dir[k];
            }
        }

        // ---- reverse_M0 ----
        std::vector<P> A0adj(static_cast<size_t>(N) * nlm * C, P(0));
#pragma omp parallel for schedule(static)
        for (int i = 0; i < N; ++i)
            for (int lm = 0; lm < nlm; ++lm) {
                P* out = A0adj.data() + (static_cast<size_t>(i) * nlm + lm) * C;
                for (int LM = 0; LM < nLM; ++LM) {
                    const P* g = M0g.data() + ((static_cast<size_t>(i) * nLM + LM) * nlm + lm) * C;
                    const P* a = M0adj.data() + (static_cast<size_t>(i) * nLM + LM) * C;
                    for (int k = 0; k < C; ++k) out[k] += g[k] * a[k];
                }
            }

        // ---- reverse_A0_scaled ----
        if (A0_scaled)
            reverse_scale(splA0, N, first.data(), types, neigh_types, xyz, r, A0.data(), A0adj.data(), forces);

        // ---- reverse_A0_streamed ----
#pragma omp parallel
        {
            std::vector<P> Phi0adj(static_cast<size_t>(nlm) * C), rad(C), drad(C);
#pragma omp for schedule(dynamic, 16)
            for (int i = 0; i < N; ++i) {
                for (int l = 0; l <= lmax; ++l) {
                    const P* W = A0W.data() + (static_cast<size_t>(types[i]) * (lmax + 1) + l) * C * C;
                    for (int lm = l * l; lm < (l + 1) * (l + 1); ++lm) {
                        const P* a = A0adj.data() + (static_cast<size_t>(i) * nlm + lm) * C;
                        P* out = Phi0adj.data() + static_cast<size_t>(lm) * C;
                        for (int ki = 0; ki < C; ++ki) {
                            const P* w = W + static_cast<size_t>(ki) * C;
                            P acc = 0;
                            for (int ko = 0; ko < C; ++ko) acc += a[ko] * w[ko];
                            out[ki] = acc;
                        }
                    }
                }
                for (long long e = first[i]; e < first[i + 1]; ++e) {
                    if (!(static_cast<P>(r[e]) < rc)) continue;
                    const auto& sp = spl0[pair_index(types[i], neigh_types[e])];
                    int iv;
                    P x;
                    sp.point(static_cast<P>(r[e]), iv, x);
                    const P* c = sp.coef(iv);
                    const P xx = x * x, xxx = xx * x;
                    const P dx = static_cast<P>(xyz[3 * e] / r[e]);
                    const P dy = static_cast<P>(xyz[3 * e + 1] / r[e]);
                    const P dz = static_cast<P>(xyz[3 * e + 2] / r[e]);
                    const P* Ye = Y.data() + e * nlm;
                    const P* Ge = Yg.data() + e * 3 * nlm;
                    const P* h0 = H0.data() + static_cast<size_t>(neigh_types[e]) * C;
                    P fx = 0, fy = 0, fz = 0;
                    for (int l = 0; l <= lmax; ++l) {
                        for (int k = 0; k < C; ++k) {
                            const int f = l * C + k;
                            rad[k] = c[f] + c[sp.nfn + f] * x + c[2 * sp.nfn + f] * xx +
                                     c[3 * sp.nfn + f] * xxx;
                            // the reference forms the derivative with double literals
                            // (cubic_spline_set.cpp:71-73), i.e. in double
                            drad[k] = static_cast<P>(c[sp.nfn + f] + 2.0 * c[2 * sp.nfn + f] * x +
                                                     3.0 * c[3 * sp.nfn + f] * xx);
                        }
                        for (int lm = l * l; lm < (l + 1) * (l + 1); ++lm) {
                            const P y = Ye[lm];
                            const P gx = Ge[lm], gy = Ge[nlm + lm], gz = Ge[2 * nlm + lm];
                            const P* adj = Phi0adj.data() + static_cast<size_t>(lm) * C;
                            for (int k = 0; k < C; ++k) {
                                const P radial_force = drad[k] * y * h0[k];
                                const P angular_force = rad[k] * h0[k];
                                const P a = adj[k];
                                fx -= a * (dx * radial_force + angular_force * gx);
                                fy -= a * (dy * radial_force + angular_force * gy);
                                fz -= a * (dz * radial_force + angular_force * gz);
                            }
                        }
                    }
                    forces[3 * e] += fx;
                    forces[3 * e + 1] += fy;
                    forces[3 * e + 2] += fz;
                }
            }
        }
    }

    // Per-l block products over nodes: out[i, l-block] = in[i, l-block] W_l
    // (or W_l^T when transpose is set), W_l of shape C x C.
    void gemm_blocks(int N, int nrows, int lblocks, const P* in, const P* W, P* out, bool transpose)
    {
#pragma omp parallel for schedule(static)
        for (int i = 0; i < N; ++i)
            for (int l = 0; l <= lblocks; ++l) {
                const P* Wl = W + static_cast<size_t>(l) * C * C;
                for (int lm = l * l; lm < (l + 1) * (l + 1); ++lm) {
                    const P* a = in + (static_cast<size_t>(i) * nrows + lm) * C;
                    P* o = out + (static_cast<size_t>(i) * nrows + lm) * C;
                    if (!transpose) {
                        for (int ko = 0; ko < C; ++ko) o[ko] = 0;
                        for (int ki = 0; ki < C; ++ki) {
                            const P v = a[ki];
                            const P* w = Wl + static_cast<size_t>(ki) * C;
                            for (int ko = 0; ko < C; ++ko) o[ko] += v * w[ko];
                        }
                    } else {
                        for (int ki = 0; ki < C; ++ki) {
                            const P* w = Wl + static_cast<size_t>(ki) * C;
                            P acc = 0;
                            for (int ko = 0; ko < C; ++ko) acc += a[ko] * w[ko];
                            o[ki] = acc;
                        }
                    }
                }
            }
    }
};

template <typename P>
void* create(const Spec* spec)
{
    try {
        return new Oracle<P>(*spec);
    } catch (const std::exception& e) {
        g_last_error = e.what();
        return nullptr;
    }
}

template <typename P>
int compute(void* handle, int N, const int* types, const int* num_neigh, const int* neigh_idx,
            const int* neigh_types, const double* xyz, const double* r, double* energies,
            double* forces, int num_threads)
{
    try {
        static_cast<Oracle<P>*>(handle)->compute(N, types, num_neigh, neigh_idx, neigh_types, xyz,
                                                 r, energies, forces, num_threads);
        return 0;
    } catch (const std::exception& e) {
        g_last_error = e.what();
        return 1;
    }
}

}  // namespace

extern "C" {

const char* oracle_mace_last_error() { return g_last_error.c_str(); }

void* oracle_mace_create_f32(const Spec* spec) { return create<float>(spec); }
void* oracle_mace_create_f64(const Spec* spec) { return create<double>(spec); }
void oracle_mace_destroy_f32(void* h) { delete static_cast<Oracle<float>*>(h); }
void oracle_mace_destroy_f64(void* h) { delete static_cast<Oracle<double>*>(h); }

int oracle_mace_compute_f32(void* h, int N, const int* types, const int* num_neigh,
                            const int* neigh_idx, const int* neigh_types, const double* xyz,
                            const double* r, double* energies, double* forces, int num_threads)
{
    return compute<float>(h, N, types, num_neigh, neigh_idx, neigh_types, xyz, r, energies, forces,
                          num_threads);
}

int oracle_mace_compute_f64(void* h, int N, const int* types, const int* num_neigh,
                            const int* neigh_idx, const int* neigh_types, const double* xyz,
                            const double* r, double* energies, double* forces, int num_threads)
{
    return compute<double>(h, N, types, num_neigh, neigh_idx, neigh_types, xyz, r, energies, forces,
                           num_threads);
}

// The oracle's ZBL pair term (value, d/dr) at n distances; 0 on success.
int oracle_zbl_pair(double a_exp, double a_prefactor, const double* c, int num_radii, const double* radii, int p,
                    int Zu, int Zv, long long n, const double* r, double* value, double* gradient)
{
    try {
        for (long long i = 0; i < n; ++i) zbl_pair_term(a_exp, a_prefactor, c, radii, num_radii, p, Zu, Zv, r[i],
                                                         value[i], gradient[i]);
        return 0;
    } catch (const std::exception& e) {
        g_last_error = e.what();
        return 1;
    }
}

// Harmonics of edge vectors as the oracle forms them in compute():
// Y [n][num_lm] and dY/d(x,y,z) [n][3][num_lm], double precision.
void oracle_harmonics(int lmax, long long n, const double* xyz, double* Y, double* dY)
{
    const int nlm = (lmax + 1) * (lmax + 1);
    for (long long e = 0; e < n; ++e) {
        const double ex = xyz[3 * e], ey = xyz[3 * e + 1], ez = xyz[3 * e + 2];
        const double rr = std::sqrt(ex * ex + ey * ey + ez * ez);
        double v[16], gx[16], gy[16], gz[16];
        double* Ye = Y + e * nlm;
        double* Ge = dY + e * 3 * nlm;
        if (rr == 0.0) {
            for (int lm = 0; lm < nlm; ++lm) {
                Ye[lm] = lm == 0 ? 1.0 : 0.0;
                Ge[lm] = Ge[nlm + lm] = Ge[2 * nlm + lm] = 0.0;
            }
            continue;
        }
        const double u0 = ez / rr, u1 = ex / rr, u2 = ey / rr;
        real_harmonics<double>(lmax, u0, u1, u2, v, gx, gy, gz);
        const double norm = 3.5449077018110318;
        for (int l = 0; l <= lmax; ++l)
            for (int lm = l * l; lm < (l + 1) * (l + 1); ++lm) {
                Ye[lm] = norm * v[lm];
                Ge[lm] = norm * (gy[lm] - l * v[lm] * u1) / rr;
                Ge[nlm + lm] = norm * (gz[lm] - l * v[lm] * u2) / rr;
                Ge[2 * nlm + lm] = norm * (gx[lm] - l * v[lm] * u0) / rr;
            }
    }
}

// The oracle's cubic Hermite spline set (double): values and derivatives of
// nfn functions at n points.  values/derivs are nodal [nfn][nodes].
void oracle_spline_eval(double h, double x0, int nodes, int nfn, const double* values, const double* derivs,
                        long long n, const double* r, double* out_value, double* out_deriv)
{
    SplineSet<double> sp;
    sp.build(h, x0, nodes, nfn, values, derivs, h);
    for (long long e = 0; e < n; ++e) {
        int iv;
        double x;
        sp.point(r[e], iv, x);
        const double* c = sp.coef(iv);
        for (int f = 0; f < nfn; ++f) {
            out_value[e * nfn + f] = c[f] + c[nfn + f] * x + c[2 * nfn + f] * x * x + c[3 * nfn + f] * x * x * x;
            out_deriv[e * nfn + f] = c[nfn + f] + 2.0 * c[2 * nfn + f] * x + 3.0 * c[3 * nfn + f] * x * x;
        }
    }
}

// The oracle's polynomial (value and gradient) of monomials of degree 1..3.
double oracle_poly_eval(int num_terms, const int* degree, const int* index, const double* coef, int nvar,
                        const double* x, double* grad)
{
    std::vector<char> used(std::max(num_terms, 1));
    Oracle<double>::first_terms(degree, index, 0, num_terms, used.data());
    return Oracle<double>::poly(coef, degree, index, used.data(), 0, num_terms, x, grad, nvar);
}

// Atom forces F_a = sum_{e: src=a} f_e - sum_{e: recv=a} f_e and stress
// sigma[3a+b] = -(1/V) sum_e f_e[a] xyz_e[b]
// (mace_kokkos_evaluate.cpp:87-106, 156-186), serial in edge order.
void oracle_reduce(int N, const int* num_neigh, const int* neigh_idx, const double* forces,
                   const double* xyz, double volume, double* atom_forces, double* stress)
{
    for (int i = 0; i < 3 * N; ++i) atom_forces[i] = 0.0;
    for (int c = 0; c < 9; ++c) stress[c] = 0.0;
    long long e = 0;
    const double scale = -1.0 / volume;
    for (int i = 0; i < N; ++i)
        for (int j = 0; j < num_neigh[i]; ++j, ++e) {
            const int s = neigh_idx[e];
            for (int c = 0; c < 3; ++c) {
                atom_forces[3 * s + c] += forces[3 * e + c];
                atom_forces[3 * i + c] -= forces[3 * e + c];
            }
            for (int c = 0; c < 9; ++c) stress[c] += scale * forces[3 * e + c / 3] * xyz[3 * e + c % 3];
        }
}

}  // extern "C"
