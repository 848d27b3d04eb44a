// Test infrastructure only: a C-ABI driver around the reference's own
// CubicSplineSetT (libsymmetrix/source/cubic_spline_set.cpp, compiled from
// /root/reference by oracle/Makefile's `ref` target into oracle/_ref/), so the
// oracle's spline restatement can be checked against the reference code.
// Nothing in the product links or loads this.
#include <exception>
#include <span>
#include <vector>

#include "cubic_spline_set.hpp"

namespace {

template <typename P>
int evaluate(P h, P x0, int nfn, int nodes, const double* values, const double* derivs, int npoints,
             const double* r, double* out_values, double* out_derivs)
{
    try {
        std::vector<std::vector<P>> v(nfn, std::vector<P>(nodes)), d(nfn, std::vector<P>(nodes));
        for (int f = 0; f < nfn; ++f)
            for (int i = 0; i < nodes; ++i) {
                v[f][i] = static_cast<P>(values[static_cast<std::size_t>(f) * nodes + i]);
                d[f][i] = static_cast<P>(derivs[static_cast<std::size_t>(f) * nodes + i]);
            }
        CubicSplineSetT<P> set(h, v, d, x0);
        std::vector<P> val(nfn), der(nfn);
        for (int p = 0; p < npoints; ++p) {
            set.evaluate_derivs(static_cast<P>(r[p]), std::span<P>(val), std::span<P>(der));
            for (int f = 0; f < nfn; ++f) {
                out_values[static_cast<std::size_t>(p) * nfn + f] = val[f];
                out_derivs[static_cast<std::size_t>(p) * nfn + f] = der[f];
            }
        }
        return 0;
    } catch (const std::exception&) {
        return 1;
    }
}

}  // namespace

// values, derivs: [nfn][nodes]; outputs [npoints][nfn]; precision 8 = double, 4 = float
extern "C" int ref_spline_eval(int precision, double h, double x0, int nfn, int nodes, const double* values,
                               const double* derivs, int npoints, const double* r, double* out_values,
                               double* out_derivs)
{
    if (precision == 8)
        return evaluate<double>(h, x0, nfn, nodes, values, derivs, npoints, r, out_values, out_derivs);
    return evaluate<float>(static_cast<float>(h), static_cast<float>(x0), nfn, nodes, values, derivs, npoints, r,
                           out_values, out_derivs);
}
