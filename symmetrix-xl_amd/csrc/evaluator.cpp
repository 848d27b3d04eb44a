// MI355X MACE evaluator host code (see evaluator.hpp).
#include "evaluator.hpp"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <map>
#include <numeric>
#include <stdexcept>
#include <thread>

#include "poly_shapes.inc"
#include "r1_shapes.inc"

namespace sxl {

namespace {

void hip_check(hipError_t err, const char* what)
{
    if (err != hipSuccess)
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(err));
}

// Copies a host vector into a device buffer.  Without staging it waits, so
// the (often temporary) host vector may be released as soon as this returns;
// with staging the copy is made from a byte copy kept in *staging, which the
// caller holds until its next wait on the stream.
template <class T>
void upload(DeviceBuffer& buf, const std::vector<T>& host, hipStream_t s,
            std::vector<std::vector<unsigned char>>* staging = nullptr)
{
    buf.reserve(std::max<std::size_t>(host.size() * sizeof(T), sizeof(T)));
    if (host.empty()) return;
    const std::size_t bytes = host.size() * sizeof(T);
    const void* src = host.data();
    if (staging) {
        const auto* b = reinterpret_cast<const unsigned char*>(host.data());
        staging->emplace_back(b, b + bytes);
        src = staging->back().data();
    }
    hip_check(hipMemcpyAsync(buf.as<void>(), src, bytes, hipMemcpyHostToDevice, s), "upload");
    if (!staging) hip_check(host_fence(s), "upload");
}

std::vector<float> to_float(const double* p, std::size_t n)
{
    std::vector<float> out(n);
    for (std::size_t i = 0; i < n; ++i) out[i] = static_cast<float>(p[i]);
    return out;
}

std::vector<float> transpose(const double* p, int rows, int cols)
{
    std::vector<float> out(static_cast<std::size_t>(rows) * cols);
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c)
            out[static_cast<std::size_t>(c) * rows + r] = static_cast<float>(p[static_cast<std::size_t>(r) * cols + c]);
    return out;
}

// A row-major [rows][cols] matrix read one row per step, a column per lane,
// in runs of four rows per column: [rows / 4][cols][4] (rows a multiple of 4)
std::vector<float> runs4(const std::vector<float>& m, int rows, int cols)
{
    if (rows % 4 != 0) throw std::invalid_argument("runs of four rows need a row count divisible by 4");
    std::vector<float> out(m.size());
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c)
            out[(static_cast<std::size_t>(r / 4) * cols + c) * 4 + r % 4] = m[static_cast<std::size_t>(r) * cols + c];
    return out;
}

// Monomial -> packed (deg | i0 << 4 | i1 << 10 | i2 << 16)
int pack_term(int degree, const int* index)
{
    return degree | (index[0] << 4) | (index[1] << 10) | (index[2] << 16);
}

struct CompiledPoly {
    int nt = 0;
    const unsigned char *out = nullptr, *deg = nullptr, *i0 = nullptr, *i1 = nullptr, *i2 = nullptr;
};

template <class P>
CompiledPoly compiled_from()
{
    return {P::NT, P::out, P::deg, P::i0, P::i1, P::i2};
}

// Compiled monomial table of (input l_max, output L_max, correlation), if any.
CompiledPoly compiled_poly(int lin, int lout, int corr)
{
    switch (lin * 100 + lout * 10 + corr) {
    case 212: return compiled_from<PolyShape<2, 1, 2>>();
    case 313: return compiled_from<PolyShape<3, 1, 3>>();
    case 323: return compiled_from<PolyShape<3, 2, 3>>();
    case 202: return compiled_from<PolyShape<2, 0, 2>>();
    case 303: return compiled_from<PolyShape<3, 0, 3>>();
    case 222: return compiled_from<PolyShape<2, 2, 2>>();
    default: return {};
    }
}

long long term_key(int out, int deg, int i0, int i1, int i2)
{
    return static_cast<long long>(out) | (static_cast<long long>(deg) << 8) | (static_cast<long long>(i0) << 16) |
           (static_cast<long long>(i1) << 24) | (static_cast<long long>(i2) << 32);
}

}  // namespace

// Places the terms of a monomial table (grouped by output, offsets
// [outputs + 1]; the loader has already dropped exact repeats, keeping each
// monomial's first coefficient) onto the slots of the compiled table of its
// shape; the terms without a compiled slot (other monomials, a second
// permutation of one index set such as [1,0] beside [0,1]) follow as the
// runtime remainder, grouped by output in JSON order.  Compiled slots that
// the JSON does not use keep a zero coefficient.
PolyLayout poly_layout(int lin, int lout, const std::vector<int>& offsets, const std::vector<int>& degree,
                       const std::vector<int>& index, bool quad)
{
    PolyLayout L;
    L.quad = quad;
    const int nout = static_cast<int>(offsets.size()) - 1;
    const int T = offsets.back();
    int corr = 0;
    for (int d : degree) corr = std::max(corr, d);
    CompiledPoly cp = compiled_poly(lin, lout, corr);
    std::map<long long, int> slot_of;
    for (int t = 0; t < cp.nt; ++t) slot_of[term_key(cp.out[t], cp.deg[t], cp.i0[t], cp.i1[t], cp.i2[t])] = t;
    L.slot.assign(T, -1);
    std::vector<char> used(cp.nt, 0);
    int matched = 0;
    for (int o = 0; o < nout; ++o)
        for (int j = offsets[o]; j < offsets[o + 1]; ++j) {
            const int* ix = index.data() + 3 * static_cast<std::size_t>(j);
            auto it = slot_of.find(term_key(o, degree[j], ix[0], ix[1], ix[2]));
            if (it != slot_of.end() && !used[it->second]) {
                L.slot[j] = it->second;
                used[it->second] = 1;
                ++matched;
            }
        }
    if (cp.nt > 0 && 2 * matched < T) {  // the compiled table does not describe this model
        cp = CompiledPoly{};
        std::fill(L.slot.begin(), L.slot.end(), -1);
    }
    L.core = cp.nt > 0 ? corr : 0;
    L.core_terms = cp.nt;
    const int core_slots = quad ? compiled_slots(cp.nt) : cp.nt;
    L.rem_offsets.push_back(0);
    for (int o = 0; o < nout; ++o) {
        for (int j = offsets[o]; j < offsets[o + 1]; ++j) {
            if (L.slot[j] >= 0) continue;
            L.slot[j] = core_slots + static_cast<int>(L.rem_packed.size());
            L.rem_packed.push_back(pack_term(degree[j], index.data() + 3 * static_cast<std::size_t>(j)));
        }
        L.rem_offsets.push_back(static_cast<int>(L.rem_packed.size()));
    }
    L.stride = core_slots + static_cast<int>(L.rem_packed.size());
    return L;
}

namespace {

// Compiled R1 shape: validates the JSON path list against the compiled one and
// scatters the JSON CG coefficients onto the compiled term slots.
template <class S>
std::vector<float> shape_cg(const HostModel& m)
{
    if (m.num_paths() != S::NP)
        throw std::invalid_argument("Phi1 path list does not match the compiled (l_max, L_max) shape.");
    for (int p = 0; p < S::NP; ++p)
        if (m.Phi1_l[p] != S::path_lo[p] || m.Phi1_l1[p] != S::path_l1[p] ||
            m.Phi1_l2[p] != S::path_l2[p])
            throw std::invalid_argument(
                "Phi1 path list does not match the compiled (l_max, L_max) shape.");
    std::map<std::pair<int, int>, int> slot;
    for (int t = 0; t < S::NT; ++t) slot[{S::term_row[t], S::term_lme[t]}] = t;
    std::vector<double> cg(S::NT, 0.0);
    for (std::size_t j = 0; j < m.Phi1_cg.size(); ++j) {
        auto it = slot.find({m.Phi1_row[j], m.Phi1_lme[j]});
        if (it == slot.end()) {
            if (m.Phi1_cg[j] == 0.0) continue;
            throw std::invalid_argument(
                "Phi1 coupling term outside the compiled CG sparsity of this shape.");
        }
        cg[it->second] += m.Phi1_cg[j];
    }
    return std::vector<float>(cg.begin(), cg.end());
}

struct ShapeInfo {
    int nlme;
    std::vector<int> num_e, lme_off;
};

// Calls f with the compiled R1 shape of (l_max, L_max), or throws.
template <class F>
void with_r1_shape(int l_max, int L_max, F&& f)
{
    switch (l_max * 10 + L_max) {
    case 21: f(R1Shape<2, 1>{}); return;
    case 31: f(R1Shape<3, 1>{}); return;
    case 32: f(R1Shape<3, 2>{}); return;
    case 30: f(R1Shape<3, 0>{}); return;
    case 20: f(R1Shape<2, 0>{}); return;
    case 22: f(R1Shape<2, 2>{}); return;
    default:
        throw std::invalid_argument("no compiled kernels for (l_max, L_max) = (" + std::to_string(l_max) + ", " +
                                    std::to_string(L_max) +
                                    "); compiled shapes: (2,0), (2,1), (2,2), (3,0), (3,1), (3,2)");
    }
}

template <class S>
ShapeInfo shape_info()
{
    ShapeInfo s;
    s.nlme = S::NLME;
    s.num_e.assign(S::num_e, S::num_e + S::LMAX + 1);
    s.lme_off.assign(S::lme_off, S::lme_off + S::LMAX + 1);
    return s;
}

}  // namespace

const char* stage_name(int stage)
{
    static const char* names[kNumStages] = {
        "edge_geometry", "a0_forward", "m0_forward", "h1_gemm", "r1_forward", "a1_gemm", "readout",
        "a1_reverse_gemm", "r1_reverse", "h1_adjoint_gather", "h1_reverse_gemm", "m0_reverse", "a0_reverse",
        "atom_forces"};
    return stage >= 0 && stage < kNumStages ? names[stage] : "";
}

namespace {
std::atomic<std::size_t> g_device_bytes{0};
}

std::size_t device_bytes_in_use() { return g_device_bytes.load(); }

ThreadCounters& thread_counters()
{
    thread_local ThreadCounters counters;
    return counters;
}

DeviceBuffer::~DeviceBuffer() { release(); }

void DeviceBuffer::release()
{
    if (ptr_) {
        (void)hipFree(ptr_);
        g_device_bytes -= bytes_;
    }
    ptr_ = nullptr;
    bytes_ = 0;
}

void DeviceBuffer::reserve(std::size_t bytes)
{
    if (bytes <= bytes_) return;
    release();
    void* p = nullptr;
    hipError_t err = hipMalloc(&p, bytes);
    if (err != hipSuccess) {
        (void)hipGetLastError();
        throw std::runtime_error("device allocation of " + std::to_string(bytes) +
                                 " bytes failed: " + hipGetErrorString(err));
    }
    ptr_ = p;
    bytes_ = bytes;
    g_device_bytes += bytes;
    ++thread_counters().allocations;
}

PinnedBuffer::~PinnedBuffer()
{
    if (ptr_) (void)hipHostFree(ptr_);
}

void PinnedBuffer::reserve(std::size_t bytes)
{
    if (bytes <= bytes_) return;
    if (ptr_) (void)hipHostFree(ptr_);
    ptr_ = nullptr;
    bytes_ = 0;
    void* p = nullptr;
    const hipError_t err = hipHostMalloc(&p, bytes, hipHostMallocDefault);
    if (err != hipSuccess) {
        (void)hipGetLastError();
        throw std::runtime_error("pinned host allocation of " + std::to_string(bytes) +
                                 " bytes failed: " + hipGetErrorString(err));
    }
    ptr_ = p;
    bytes_ = bytes;
    ++thread_counters().allocations;
}

void Evaluator::account_preparation(const CallStart& start)
{
    stats_.preparation_fences += static_cast<long long>(thread_counters().fences - start.counters.fences);
    stats_.last_graph_prepare_ms =
        std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - start.time).count();
}

void Evaluator::wait(const char* what)
{
    hip_check(host_fence(stream_), what);
    staged_.clear();
}

void Evaluator::account_evaluation(const CallStart& start)
{
    const ThreadCounters& now = thread_counters();
    stats_.last_evaluation_launches = static_cast<long long>(now.launches - start.counters.launches);
    stats_.last_evaluation_allocations = static_cast<long long>(now.allocations - start.counters.allocations);
    stats_.last_evaluation_fences = static_cast<long long>(now.fences - start.counters.fences);
    stats_.evaluation_fences += stats_.last_evaluation_fences;
}

Evaluator::Evaluator(const std::string& model_path, const std::string& head)
    : model_(HostModel::load(model_path, head))
{
    int devices = 0;
    if (hipGetDeviceCount(&devices) != hipSuccess || devices == 0) {
        (void)hipGetLastError();
        throw std::runtime_error("no HIP device is available");
    }
    hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "stream create");
    {
        int device = 0;
        hip_check(hipGetDevice(&device), "device query");
        hip_check(hipDeviceGetAttribute(&compute_units_, hipDeviceAttributeMultiprocessorCount, device),
                  "compute unit query");
    }
    C_ = model_.channels;
    nlm_ = model_.num_lm;
    nLM_ = model_.num_LM;
    ShapeInfo info;
    with_r1_shape(model_.l_max, model_.L_max, [&](auto shape) { info = shape_info<decltype(shape)>(); });
    nlme_ = info.nlme;
    num_e_ = info.num_e;
    lme_off_ = info.lme_off;
    if (C_ % 32 != 0 || C_ > 1024)
        throw std::invalid_argument("channel count must be a multiple of 32 and at most 1024");
    // one workgroup of C threads per receiver, at most 256 threads
    if (C_ > 256) throw std::invalid_argument("channel counts above 256 are not supported yet");
    grid_.x0 = model_.grid_min;
    grid_.h = model_.spline_h;
    grid_.intervals = model_.spline_points - 1;
    grid_.r_cut = model_.r_cut;
    // test hook: a lower edge-index ceiling makes small graphs take the
    // paths of graphs past 2^31 - 1 edges
    if (const char* limit = std::getenv("SXL_EDGE_INDEX_LIMIT"); limit && limit[0]) {
        const long long v = std::atoll(limit);
        if (v > 0 && v < edge_index_limit_) edge_index_limit_ = v;
    }
    upload_static_tables();
    hip_check(host_fence(stream_), "model upload");
}

void Evaluator::set_profiling(bool enable) { set_profiling_stages(enable ? ~0u : 0u); }

void Evaluator::set_profiling_stages(unsigned mask)
{
    const bool enable = mask != 0;
    profile_mask_ = mask;
    if (enable && events_.empty()) {
        events_.resize(2 * kNumStages);
        for (auto& e : events_) hip_check(hipEventCreate(&e), "event create");
    }
    profiling_ = enable;
    for (int i = 0; i < kNumStages; ++i) {
        stage_ms_[i] = 0.0;
        stage_count_[i] = 0;
    }
}

void Evaluator::stage_times(double* ms, int* counts) const
{
    for (int i = 0; i < kNumStages; ++i) {
        if (ms) ms[i] = stage_ms_[i];
        if (counts) counts[i] = stage_count_[i];
    }
}

void Evaluator::mark(int stage, bool end)
{
    if (!profiling_ || !((profile_mask_ >> stage) & 1u)) return;
    hip_check(hipEventRecord(events_[2 * stage + (end ? 1 : 0)], stream_), "event record");
    if (end) stage_used_[stage] = true;
}

Evaluator::~Evaluator()
{
    if (stream_) (void)host_fence(stream_);
    release_replay();
    for (auto& e : events_) (void)hipEventDestroy(e);
    // buffers free themselves; the stream goes last
    A0_.release();
    if (stream_) (void)hipStreamDestroy(stream_);
}

void Evaluator::upload_static_tables()
{
    const HostModel& m = model_;
    const int L1 = m.L_max + 1;
    upload(h1w_, to_float(m.H1W.data(), m.H1W.size()), stream_);
    std::vector<float> h1wt;
    for (int l = 0; l < L1; ++l) {
        auto t = transpose(m.H1W.data() + static_cast<std::size_t>(l) * C_ * C_, C_, C_);
        h1wt.insert(h1wt.end(), t.begin(), t.end());
    }
    upload(h1wt_, h1wt, stream_);
    a1w_.clear();
    a1wt_.clear();
    for (int l = 0; l <= m.l_max; ++l) {
        a1w_.push_back(std::make_unique<DeviceBuffer>());
        a1wt_.push_back(std::make_unique<DeviceBuffer>());
        upload(*a1w_[l], to_float(m.A1W[l].data(), m.A1W[l].size()), stream_);
        upload(*a1wt_[l], transpose(m.A1W[l].data(), num_e_[l] * C_, C_), stream_);
    }
    if (m.pre_linear_up) {
        upload(p0w_, to_float(m.H1P.data(), static_cast<std::size_t>(C_) * C_), stream_);
        upload(p0wt_, transpose(m.H1P.data(), C_, C_), stream_);
    }
    if (m.first_residual) {
        upload(residual_, to_float(m.residual.data(), m.residual.size()), stream_);
        upload(residual_fused_, to_float(m.residual_fused.data(), m.residual_fused.size()), stream_);
    }
    upload(h2m1_, runs4(to_float(m.H2M1.data(), m.H2M1.size()), C_, C_), stream_);
    upload(h2m1t_, runs4(transpose(m.H2M1.data(), C_, C_), C_, C_), stream_);
    upload(q_, to_float(m.readout_q.data(), m.readout_q.size()), stream_);
    upload(w1_, to_float(m.readout_w1.data(), m.readout_w1.size()), stream_);
    upload(w2_, to_float(m.readout_w2.data(), m.readout_w2.size()), stream_);
    std::vector<float> cg;
    with_r1_shape(m.l_max, m.L_max, [&](auto shape) { cg = shape_cg<decltype(shape)>(m); });
    upload(cg_, cg, stream_);
    p0_layout_ = poly_layout(m.l_max, m.L_max, m.m0_offsets, m.m0_degree, m.m0_index, true);
    upload(p0_offsets_, p0_layout_.rem_offsets, stream_);
    upload(p0_packed_, p0_layout_.rem_packed, stream_);
    const std::vector<int> off1 = {0, static_cast<int>(m.m1_degree.size())};
    p1_layout_ = poly_layout(m.l_max, 0, off1, m.m1_degree, m.m1_index, false);
    upload(p1_offsets_, p1_layout_.rem_offsets, stream_);
    upload(p1_packed_, p1_layout_.rem_packed, stream_);
}

PolyArgs Evaluator::poly_args(const PolyLayout& layout, const DeviceBuffer& coef, const DeviceBuffer& offsets,
                              const DeviceBuffer& packed) const
{
    PolyArgs p;
    p.core = layout.core;
    p.stride = layout.stride;
    p.num_rem = static_cast<int>(layout.rem_packed.size());
    p.rem_offsets = offsets.as<int>();
    p.rem_packed = packed.as<int>();
    p.coef = coef.as<float>();
    return p;
}

// Radial spline tables and per-type weights of the active element types
// (reference MACECPU::prepare_active_types, mace.cpp:118-213, with H0 and
// A0_W folded into the layer-0 splines per ordered pair as the reference's
// device path does, mace_kokkos_factorized_lifecycle.cpp:3990-4046).
void Evaluator::prepare_active_types(const std::vector<int>& node_types)
{
    std::vector<int> types(node_types.begin(), node_types.end());
    std::sort(types.begin(), types.end());
    types.erase(std::unique(types.begin(), types.end()), types.end());
    if (types.empty()) throw std::invalid_argument("MACE compact radial cache requires at least one active type.");
    for (int t : types)
        if (t < 0 || t >= model_.num_elements) throw std::out_of_range("MACE active type index is out of range.");
    if (types == active_types_) return;
    const HostModel& m = model_;
    const int na = static_cast<int>(types.size());
    if (na * na > 0xffff) throw std::invalid_argument("too many active element types");
    const int P = m.spline_points, NI = P - 1, NL = m.l_max + 1, NP = m.num_paths();
    const double h = m.spline_h;
    // nodal tables per unordered pair; one table for all pairs when the
    // radial functions do not depend on the element types (no distance
    // transform with per-element radii): the kernels then index table 0
    const int npairs = shared_pair_tables() ? 1 : na * (na + 1) / 2;
    std::vector<std::vector<double>> r0v(npairs), r0d(npairs), r1v(npairs), r1d(npairs);
    std::vector<std::pair<int, int>> pair_types;
    for (int a = 0; a < na; ++a)
        for (int b = a; b < na; ++b) pair_types.push_back({a, b});
    pair_types.resize(npairs);
    auto tabulate = [&](int p) {
        const int ti = types[pair_types[p].first], tj = types[pair_types[p].second];
        m.radial_tables(m.R0, ti, tj, r0v[p], r0d[p]);
        m.radial_tables(m.R1, ti, tj, r1v[p], r1d[p]);
    };
    const int nthreads = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    {
        std::vector<std::thread> pool;
        for (int w = 0; w < nthreads; ++w)
            pool.emplace_back([&, w] {
                for (int p = w; p < npairs; p += nthreads) tabulate(p);
            });
        for (auto& t : pool) t.join();
    }
    auto hermite = [&](const std::vector<double>& v, const std::vector<double>& d, int fn, int iv,
                       double* c4) {
        const double v0 = v[static_cast<std::size_t>(fn) * P + iv], v1 = v[static_cast<std::size_t>(fn) * P + iv + 1];
        const double d0 = d[static_cast<std::size_t>(fn) * P + iv], d1 = d[static_cast<std::size_t>(fn) * P + iv + 1];
        c4[0] = v0;
        c4[1] = d0;
        c4[2] = (-3.0 * v0 - 2.0 * h * d0 + 3.0 * v1 - h * d1) / (h * h);
        c4[3] = (2.0 * v0 + h * d0 - 2.0 * v1 + h * d1) / (h * h * h);
    };
    // R1 table: [pair_u][iv][p][k][q]
    std::vector<float> r1(static_cast<std::size_t>(npairs) * NI * 4 * NP * C_);
    for (int pu = 0; pu < npairs; ++pu)
        for (int iv = 0; iv < NI; ++iv)
            for (int p = 0; p < NP; ++p)
                for (int k = 0; k < C_; ++k) {
                    double c4[4];
                    hermite(r1v[pu], r1d[pu], p * C_ + k, iv, c4);
                    for (int q = 0; q < 4; ++q)
                        r1[(((static_cast<std::size_t>(pu) * NI + iv) * NP + p) * C_ + k) * 4 + q] =
                            static_cast<float>(c4[q]);
                }
    // R0 folded: [pair_o][iv][l][k'][q] = sum_k c[iv][q][l*C+k] H0[tj][k] A0W[ti][l][k][k']
    std::vector<float> r0f(static_cast<std::size_t>(na) * na * NI * 4 * NL * C_);
    auto fold = [&](int po) {
        const int ai = po / na, aj = po % na;
        const int ti = types[ai], tj = types[aj];
        const int pu = npairs == 1 ? 0
                       : ai <= aj ? ai * (2 * na - ai - 1) / 2 + aj
                                  : aj * (2 * na - aj - 1) / 2 + ai;
        std::vector<double> u(C_), out(C_);
        for (int iv = 0; iv < NI; ++iv)
            for (int q = 0; q < 4; ++q)
                for (int l = 0; l < NL; ++l) {
                    for (int k = 0; k < C_; ++k) {
                        double c4[4];
                        hermite(r0v[pu], r0d[pu], l * C_ + k, iv, c4);
                        u[k] = c4[q] * m.H0[static_cast<std::size_t>(tj) * C_ + k];
                    }
                    std::fill(out.begin(), out.end(), 0.0);
                    const double* W = m.A0W.data() + (static_cast<std::size_t>(ti) * NL + l) * C_ * C_;
                    for (int k = 0; k < C_; ++k) {
                        const double uk = u[k];
                        const double* w = W + static_cast<std::size_t>(k) * C_;
                        for (int ko = 0; ko < C_; ++ko) out[ko] += uk * w[ko];
                    }
                    float* dst = r0f.data() + (((static_cast<std::size_t>(po) * NI + iv) * NL + l) * C_) * 4 + q;
                    for (int ko = 0; ko < C_; ++ko) dst[4 * ko] = static_cast<float>(out[ko]);
                }
    };
    {
        std::vector<std::thread> pool;
        for (int w = 0; w < nthreads; ++w)
            pool.emplace_back([&, w] {
                for (int po = w; po < na * na; po += nthreads) fold(po);
            });
        for (auto& t : pool) t.join();
    }
    upload(r1_, r1, stream_, &staged_);
    // the layer-0 tables are kept on the host; place_layer0_tables() puts the
    // one the selected plan reads on the device
    host_r0f_ = std::move(r0f);
    r0f_.release();
    // the unfolded layer-0 table and its per-type factors (kA0FoldedTableBytes);
    // SXL_A0_UNFOLDED=1 / 0 forces the choice (tests)
    const char* force_unfolded = std::getenv("SXL_A0_UNFOLDED");
    a0_unfold_ = force_unfolded && force_unfolded[0] ? force_unfolded[0] == '1'
                                                     : host_r0f_.size() * sizeof(float) > kA0FoldedTableBytes;
    if (a0_unfold_) {
        std::vector<float> r0u(static_cast<std::size_t>(npairs) * NI * 4 * NL * C_);
        for (int pu = 0; pu < npairs; ++pu)
            for (int iv = 0; iv < NI; ++iv)
                for (int l = 0; l < NL; ++l)
                    for (int k = 0; k < C_; ++k) {
                        double c4[4];
                        hermite(r0v[pu], r0d[pu], l * C_ + k, iv, c4);
                        for (int q = 0; q < 4; ++q)
                            r0u[(((static_cast<std::size_t>(pu) * NI + iv) * NL + l) * C_ + k) * 4 + q] =
                                static_cast<float>(c4[q]);
                    }
        std::vector<float> h0(static_cast<std::size_t>(na) * C_);
        std::vector<float> w(static_cast<std::size_t>(na) * NL * C_ * C_), wt(w.size());
        for (int a = 0; a < na; ++a) {
            for (int k = 0; k < C_; ++k)
                h0[static_cast<std::size_t>(a) * C_ + k] =
                    static_cast<float>(m.H0[static_cast<std::size_t>(types[a]) * C_ + k]);
            for (int l = 0; l < NL; ++l) {
                const double* W = m.A0W.data() + (static_cast<std::size_t>(types[a]) * NL + l) * C_ * C_;
                const std::size_t base = (static_cast<std::size_t>(a) * NL + l) * C_ * C_;
                for (int k = 0; k < C_; ++k)
                    for (int ko = 0; ko < C_; ++ko) {
                        const float v = static_cast<float>(W[static_cast<std::size_t>(k) * C_ + ko]);
                        w[base + static_cast<std::size_t>(k) * C_ + ko] = v;   // reverse: out[k] += in[ko] w[k][ko]
                        wt[base + static_cast<std::size_t>(ko) * C_ + k] = v;  // forward: out[ko] += in[k] wt[ko][k]
                    }
            }
        }
        host_r0u_ = std::move(r0u);
        host_h0_ = std::move(h0);
        host_a0w_ = std::move(w);
        host_a0wt_ = std::move(wt);
    } else {
        host_r0u_.clear();
        host_h0_.clear();
        host_a0w_.clear();
        host_a0wt_.clear();
    }
    r0u_.release();
    h0s_.release();
    a0w_.release();
    a0wt_.release();
    // the second-interaction forward of a 256-channel model runs in 64-channel
    // slices, one slice per XCD, when its coefficient table is far beyond one
    // XCD's L2 (4 MiB), and so does the reverse of the (3, 2) shape
    // (SXL_R1_REVERSE_SLICES = 1 or C / 64 forces the reverse's count: tests)
    r1_slices_ = 1;
    if (C_ == 256 && r1.size() * sizeof(float) > kR1SliceTableBytes) r1_slices_ = C_ / 64;
    r1_rev_slices_ = r1_reverse_sliceable(model_.l_max, model_.L_max, C_, r1_slices_) ? r1_slices_ : 1;
    if (const char* force = std::getenv("SXL_R1_REVERSE_SLICES"); force && force[0]) {
        const int n = std::atoi(force);
        if (!r1_reverse_sliceable(model_.l_max, model_.L_max, C_, n))
            throw std::invalid_argument("SXL_R1_REVERSE_SLICES=" + std::string(force) +
                                        " does not fit this model (1, or 64-channel slices of the l_max 3, L_max 2 "
                                        "shape)");
        r1_rev_slices_ = n;
    }
    // density-normalisation splines per unordered pair: [pair_u][iv][4]
    auto density_table = [&](const RadialNetwork& net, DeviceBuffer& out) {
        std::vector<float> table(static_cast<std::size_t>(npairs) * NI * 4);
        for (int pu = 0; pu < npairs; ++pu) {
            std::vector<double> v, d;
            m.radial_tables(net, types[pair_types[pu].first], types[pair_types[pu].second], v, d);
            for (int iv = 0; iv < NI; ++iv) {
                double c4[4];
                hermite(v, d, 0, iv, c4);
                for (int q = 0; q < 4; ++q)
                    table[(static_cast<std::size_t>(pu) * NI + iv) * 4 + q] = static_cast<float>(c4[q]);
            }
        }
        upload(out, table, stream_, &staged_);
    };
    if (m.A0_scaled) density_table(m.A0net, dens0_);
    if (m.A1_scaled) density_table(m.A1net, dens1_);
    // ZBL per ordered active pair (receiver, source), zbl_kokkos.cpp:37-52
    if (m.has_zbl) {
        std::vector<double> inv_a(na * na), pref(na * na), rmax(na * na);
        for (int ai = 0; ai < na; ++ai)
            for (int aj = 0; aj < na; ++aj) {
                const int zu = m.atomic_numbers[types[ai]], zv = m.atomic_numbers[types[aj]];
                const double denominator = std::pow(static_cast<double>(zu), m.zbl_a_exp) +
                                           std::pow(static_cast<double>(zv), m.zbl_a_exp);
                inv_a[ai * na + aj] = denominator / (m.zbl_a_prefactor * 0.529);
                pref[ai * na + aj] = 14.3996 * static_cast<double>(zu * zv);
                rmax[ai * na + aj] = m.zbl_radii[zu] + m.zbl_radii[zv];
            }
        upload(zbl_inverse_a_, inv_a, stream_, &staged_);
        upload(zbl_prefactor_, pref, stream_, &staged_);
        upload(zbl_rmax_, rmax, stream_, &staged_);
    }
    // per active type tables
    std::vector<int> type_active(m.num_elements, -1);
    for (int a = 0; a < na; ++a) type_active[types[a]] = a;
    upload(type_active_, type_active, stream_, &staged_);
    std::vector<float> p0c, p1c, h2m0, h2m0t;
    std::vector<double> e0;
    // coefficients per active type on the slots of the polynomial layouts:
    // [slot][C], or for a quad layout the compiled slots in runs of four per
    // channel ([slot / 4][C][4], one 16-byte load per lane for four terms)
    auto place = [&](const PolyLayout& L, const std::vector<double>& coef, int t, std::vector<float>& out) {
        const std::size_t T = L.slot.size();
        const std::size_t base = out.size();
        out.resize(base + static_cast<std::size_t>(L.stride) * C_, 0.0f);
        for (std::size_t j = 0; j < T; ++j) {
            const std::size_t s = static_cast<std::size_t>(L.slot[j]);
            for (int k = 0; k < C_; ++k) {
                const std::size_t at =
                    L.quad && static_cast<int>(s) < L.core_terms ? (s / 4 * C_ + k) * 4 + s % 4 : s * C_ + k;
                out[base + at] = static_cast<float>(coef[(static_cast<std::size_t>(t) * T + j) * C_ + k]);
            }
        }
    };
    for (int a = 0; a < na; ++a) {
        const int t = types[a];
        place(p0_layout_, m.m0_coef, t, p0c);
        place(p1_layout_, m.m1_coef, t, p1c);
        auto hm = runs4(to_float(m.H2M0.data() + static_cast<std::size_t>(t) * C_ * C_,
                                 static_cast<std::size_t>(C_) * C_),
                        C_, C_);
        h2m0.insert(h2m0.end(), hm.begin(), hm.end());
        auto hmt = runs4(transpose(m.H2M0.data() + static_cast<std::size_t>(t) * C_ * C_, C_, C_), C_, C_);
        h2m0t.insert(h2m0t.end(), hmt.begin(), hmt.end());
        e0.push_back(m.atomic_energies[t]);
    }
    upload(p0_coef_, p0c, stream_, &staged_);
    upload(p1_coef_, p1c, stream_, &staged_);
    upload(h2m0_, h2m0, stream_, &staged_);
    upload(h2m0t_, h2m0t, stream_, &staged_);
    upload(e0_, e0, stream_, &staged_);
    active_types_ = types;
}

void Evaluator::check_generation(std::uint64_t generation) const
{
    if (generation == 0 || generation != generation_)
        throw std::invalid_argument("stale or unknown graph generation token");
}

void Evaluator::allocate_workspace()
{
    const std::size_t N = std::max(num_nodes_, 1);
    const std::size_t E = std::max<long long>(num_edges_, 1);
    const std::size_t f = sizeof(float);
    const bool tiled = tile_receivers_ > 0;
    // receiver-indexed work arrays span one tile (the whole graph untiled)
    const std::size_t NT = tiled ? static_cast<std::size_t>(tile_receivers_) : N;
    std::size_t ET = E;
    if (tiled) {
        ET = 1;
        for (int t = 0; t < num_tiles_; ++t)
            ET = std::max<std::size_t>(ET, tile_first_edge_[t + 1] - tile_first_edge_[t]);
    }
    if (tiled || model_.pre_linear_up)
        M0s_.reserve(N * C_ * f);
    else
        M0s_.release();
    A0_.reserve(NT * nlm_ * C_ * f);
    if (a0_unfolded())
        A0pre_.reserve(N * nlm_ * C_ * f);
    else
        A0pre_.release();
    M0_.reserve(NT * nLM_ * C_ * f);
    Phi1_.reserve(NT * nlme_ * C_ * f);
    A1_.reserve(NT * nlm_ * C_ * f);
    A1adj_.reserve(NT * nlm_ * C_ * f);
    msg_.reserve(ET * nLM_ * C_ * f);
    if (r1_rev_slices_ > 1)
        rpart_.reserve(ET * r1_rev_slices_ * 3 * sizeof(double));
    else
        rpart_.release();
    // graph-wide
    H1_.reserve(N * nLM_ * C_ * f);
    H1adj_.reserve(N * nLM_ * C_ * f);
    // the tiled plan writes the readout's direct adjoint over the scalar M0
    // block (M0s_): the readout reads a node's block before it writes that
    // node's adjoint, and nothing reads the block afterwards
    if (tiled)
        direct_.release();
    else
        direct_.reserve(N * C_ * f);
    if (model_.A1_scaled) {
        scale1_.reserve(N * f);
        dot1_.reserve(N * f);
    }
    energies_.reserve(N * sizeof(double));
    atom_forces_.reserve(N * 3 * sizeof(double));
    // totals partials: nodes and edges of the graph (untiled) or of one tile
    partials_.reserve(static_cast<std::size_t>(reduce_totals_partials(num_nodes_, static_cast<int>(ET))) * 10 *
                      sizeof(double));
    // [0] energy, [1..9] stress, [12] max |disp|^2, [13] invalid edges,
    // [16..25] tiled plan: -sum f (x) xyz accumulated over the tiles
    totals_.reserve(32 * sizeof(double));
    if (tiled) {
        // per-edge state lives in the tile arena
        forces_.release();
        xyz_.release();
        r_.release();
        tile_xyz_.reserve(ET * 3 * sizeof(double));
        tile_r_.reserve(ET * sizeof(double));
        tile_pair_.reserve(ET * sizeof(int));
        tile_forces_.reserve(ET * 3 * sizeof(double));
    } else {
        tile_xyz_.release();
        tile_r_.release();
        tile_pair_.release();
        tile_forces_.release();
        forces_.reserve(E * 3 * sizeof(double));
        xyz_.reserve(E * 3 * sizeof(double));
        r_.reserve(E * sizeof(double));
    }
}

namespace {
// Device memory the planner refuses to plan for: the estimate of the plan
// exceeds everything the device could give this evaluator (std::bad_alloc,
// so callers see an allocation error, with the planner's figures).
class PlanMemoryError : public std::bad_alloc {
public:
    explicit PlanMemoryError(std::string message) : message_(std::move(message)) {}
    const char* what() const noexcept override { return message_.c_str(); }

private:
    std::string message_;
};
}  // namespace

// Execution plan of the graph being prepared, from its receiver offsets
// (host_first_) before its edges are written.  The untiled plan indexes
// edges graph-wide in int32 and takes at most edge_index_limit_ edges; the
// tiled plan indexes them per tile.  With fixed workspace allowed, the graph
// is tiled when a receiver limit below N is set, when the untiled work
// arrays would not fit the memory budget, or when its edges exceed the
// untiled plan's index (tiles of kDefaultTileReceivers by default).  A tiled
// plan whose estimate exceeds all the memory the device could give is
// refused here, before the edges are written.
void Evaluator::select_plan()
{
    tile_receivers_ = 0;
    num_tiles_ = 0;
    tile_first_edge_.clear();
    tile_run_offsets_.clear();
    const int N = num_nodes_;
    const long long E = num_edges_;
    static const char* kSpeed = "mh0-direct-speed";
    static const char* kTiled = "mh0-dual-layer-tiled-v1";

    ExecutionPlanReport rep;
    rep.requested_profile = plan_profile_;
    rep.selection_source = plan_debug_.empty() ? "native_request" : "debug_override";
    const std::vector<long long>& first = host_first_;
    const int T = receiver_limit_ > 0 ? receiver_limit_ : kDefaultTileReceivers;
    const int tiles = N > 0 ? static_cast<int>((static_cast<long long>(N) + T - 1) / T) : 0;
    long long tile_edges = 0;
    for (long long t0 = 0; t0 < N; t0 += T)
        tile_edges = std::max<long long>(tile_edges, first[std::min<long long>(N, t0 + T)] - first[t0]);
    // runs (distinct sources per tile): counted by the device build's count
    // pass or by count_tile_runs; otherwise at least one per node
    long long runs = N;
    if (static_cast<int>(tile_runs_.size()) == tiles && tiles > 0)
        runs = std::accumulate(tile_runs_.begin(), tile_runs_.end(), 0LL);
    const std::size_t untiled = graph_bytes_estimate(false, 0) + work_bytes_estimate(N, E, false);
    const std::size_t tiled = graph_bytes_estimate(true, runs) +
                              work_bytes_estimate(std::min(T, std::max(N, 1)), tile_edges, true);
    // memory budget: free device memory plus the graph and work memory this
    // evaluator holds now (the estimates count all of a plan's memory)
    std::size_t free_bytes = 0, total_bytes = 0;
    hip_check(hipMemGetInfo(&free_bytes, &total_bytes), "memory info");
    rep.available_bytes = free_bytes + held_graph_bytes();
    // test hook: SXL_DEVICE_MEMORY_LIMIT (bytes) caps what the planner may use
    if (const char* cap = std::getenv("SXL_DEVICE_MEMORY_LIMIT"); cap && cap[0]) {
        const long long v = std::atoll(cap);
        if (v > 0) rep.available_bytes = std::min<std::size_t>(rep.available_bytes, static_cast<std::size_t>(v));
    }
    rep.reserve_bytes = rep.available_bytes / 10;
    const std::size_t budget = rep.available_bytes - rep.reserve_bytes;
    const bool tiled_permitted = allow_fixed_workspace_ || plan_debug_ == kTiled;
    const bool untiled_indexable = E <= edge_index_limit_;
    const bool tiles_indexable = tile_edges <= edge_index_limit_;
    const std::string over_index =
        "the graph's " + std::to_string(E) + " edges exceed the untiled plan's 32-bit edge index";
    rep.candidates.push_back({kSpeed, untiled_indexable, untiled,
                              !untiled_indexable ? over_index
                              : untiled <= budget ? "estimated fit"
                                                  : "exceeds advisory memory budget"});
    rep.candidates.push_back(
        {kTiled, tiled_permitted && N > T && tiles_indexable, tiled,
         !tiled_permitted  ? "fixed-workspace execution requires explicit opt-in via allow_fixed_workspace"
         : !(N > T)        ? "the graph fits in one tile of " + std::to_string(T) + " receivers"
         : !tiles_indexable ? "a tile of " + std::to_string(T) + " receivers has " + std::to_string(tile_edges) +
                                  " edges, more than one tile's 32-bit edge index"
                           : "qualified"});

    bool tile = false;
    if (plan_debug_ == kSpeed) {
        rep.selection_reason = "debug override selected the untiled plan";
    } else if (plan_debug_ == kTiled) {
        tile = N > T;
        rep.selection_reason = tile ? "debug override selected receiver tiles"
                                    : "debug override: the graph fits in one tile, untiled";
    } else if (plan_profile_ == "speed") {
        rep.selection_reason = "speed request selected the untiled plan";
    } else if (!untiled_indexable && allow_fixed_workspace_ && N > T) {
        tile = true;
        rep.selection_reason = over_index + "; tiles of " + std::to_string(T) + " receivers";
    } else if (allow_fixed_workspace_ && receiver_limit_ > 0 && N > T) {
        tile = true;
        rep.selection_reason = "receiver limit " + std::to_string(T) + " set for the tiled plan";
    } else if (untiled <= budget) {
        rep.selection_reason = "untiled estimate fits within the post-reserve budget";
    } else if (allow_fixed_workspace_ && N > T) {
        tile = true;
        rep.selection_reason = "untiled estimate exceeds the post-reserve budget; tiles of " + std::to_string(T) +
                               " receivers";
    } else {
        rep.selection_reason = "no permitted plan fits the post-reserve budget; attempting the untiled plan";
    }
    rep.selected_id = tile ? kTiled : kSpeed;
    rep.boundary_attempt = (tile ? tiled : untiled) > budget;
    rep.state = tile || untiled_indexable ? "active" : "refused";
    plan_report_ = rep;
    if (!tile) {
        if (!untiled_indexable)
            throw std::length_error("neighbor graph exceeds 32-bit edge indexing (" + std::to_string(E) +
                                    " edges); fixed-workspace (tiled) execution indexes edges per tile");
        return;
    }
    if (!tiles_indexable)
        throw std::length_error("a receiver tile of " + std::to_string(T) + " receivers has " +
                                std::to_string(tile_edges) +
                                " edges, beyond 32-bit edge indexing; set a smaller workspace receiver limit");
    if (tiled > rep.available_bytes) {
        plan_report_.state = "refused";
        throw PlanMemoryError("MACE tiled execution plan needs an estimated " + std::to_string(tiled) +
                              " bytes of device memory for " + std::to_string(N) + " atoms and " +
                              std::to_string(E) + " edges; the device can give " +
                              std::to_string(rep.available_bytes) + " bytes");
    }
    tile_receivers_ = T;
    num_tiles_ = tiles;
    tile_first_edge_.resize(num_tiles_ + 1);
    for (int t = 0; t <= num_tiles_; ++t)
        tile_first_edge_[t] = first[std::min<long long>(N, static_cast<long long>(t) * T)];
}

// Distinct edge sources of each receiver tile of T receivers, from the
// graph's sources on the device (caller graphs; the device build counts them
// in its count pass).
void Evaluator::count_tile_runs()
{
    const int N = num_nodes_;
    const int T = receiver_limit_ > 0 ? receiver_limit_ : kDefaultTileReceivers;
    const int tiles = static_cast<int>((static_cast<long long>(N) + T - 1) / T);
    DeviceBuffer last_tile, counts;
    last_tile.reserve(static_cast<std::size_t>(std::max(N, 1)) * sizeof(int));
    counts.reserve(static_cast<std::size_t>(std::max(tiles, 1)) * sizeof(int));
    hip_check(launch_fill_i32(last_tile.as<int>(), N, -1, stream_), "tile runs");
    hip_check(launch_fill_i32(counts.as<int>(), tiles, 0, stream_), "tile runs");
    for (int t = 0; t < tiles; ++t) {
        const long long base = host_first_[static_cast<std::size_t>(t) * T];
        const long long end = host_first_[std::min<long long>(N, static_cast<long long>(t + 1) * T)];
        hip_check(launch_tile_runs_mark(static_cast<int>(end - base), source_.as<int>() + base, t,
                                        last_tile.as<int>(), nullptr, nullptr, counts.as<int>() + t, stream_),
                  "tile runs");
    }
    tile_runs_.assign(tiles, 0);
    if (tiles > 0)
        hip_check(hipMemcpyAsync(tile_runs_.data(), counts.as<int>(), tiles * sizeof(int), hipMemcpyDeviceToHost,
                                 stream_),
                  "copy");
    wait("tile runs");
}

// Tiled plan, once the sources are on the device: tile-local receiver
// offsets (first_), each tile's edges grouped by source with ascending
// tile-local ids (tedge_, at the tile's first edge) and the runs (source,
// start in the tile's list, length) of every tile.
void Evaluator::build_tile_lists()
{
    const int N = num_nodes_;
    const int T = tile_receivers_;
    const int tiles = num_tiles_;
    std::vector<int> local(static_cast<std::size_t>(N) + tiles);
    for (int t = 0; t < tiles; ++t) {
        const long long lo = static_cast<long long>(t) * T;
        const int count = static_cast<int>(std::min<long long>(T, N - lo));
        for (int j = 0; j <= count; ++j)
            local[static_cast<std::size_t>(t) * (T + 1) + j] =
                static_cast<int>(host_first_[lo + j] - tile_first_edge_[t]);
    }
    upload(first_, local, stream_, &staged_);
    if (static_cast<int>(tile_runs_.size()) != tiles) count_tile_runs();
    tile_run_offsets_.assign(tiles + 1, 0);
    int max_runs = 0;
    for (int t = 0; t < tiles; ++t) {
        tile_run_offsets_[t + 1] = tile_run_offsets_[t] + tile_runs_[t];
        max_runs = std::max(max_runs, tile_runs_[t]);
    }
    const int runs = tile_run_offsets_[tiles];
    const long long E = num_edges_;
    run_source_.reserve(static_cast<std::size_t>(std::max(runs, 1)) * sizeof(int));
    run_start_.reserve((static_cast<std::size_t>(runs) + 1) * sizeof(int));
    run_length_.reserve(static_cast<std::size_t>(std::max(runs, 1)) * sizeof(int));
    tedge_.reserve(static_cast<std::size_t>(std::max<long long>(E, 1)) * sizeof(int));
    DeviceBuffer last_tile, run_of, counts, cursors, scan, scan_scratch;
    last_tile.reserve(static_cast<std::size_t>(std::max(N, 1)) * sizeof(int));
    run_of.reserve(static_cast<std::size_t>(std::max(N, 1)) * sizeof(int));
    counts.reserve(static_cast<std::size_t>(std::max(tiles, 1)) * sizeof(int));
    cursors.reserve(static_cast<std::size_t>(std::max(max_runs, 1)) * sizeof(int));
    scan.reserve((static_cast<std::size_t>(max_runs) + 1) * sizeof(long long));
    scan_scratch.reserve(scan_scratch_size(max_runs + 1) * sizeof(long long));
    hip_check(launch_fill_i32(last_tile.as<int>(), N, -1, stream_), "tile lists");
    hip_check(launch_fill_i32(counts.as<int>(), tiles, 0, stream_), "tile lists");
    for (int t = 0; t < tiles; ++t) {
        const long long base = tile_first_edge_[t];
        const int n = static_cast<int>(tile_first_edge_[t + 1] - base);
        const int nr = tile_runs_[t];
        const int off = tile_run_offsets_[t];
        const int* src = source_.as<int>() + base;
        int* start = run_start_.as<int>() + off;
        hip_check(launch_tile_runs_mark(n, src, t, last_tile.as<int>(), run_of.as<int>(),
                                        run_source_.as<int>() + off, counts.as<int>() + t, stream_),
                  "tile runs");
        hip_check(launch_fill_i32(run_length_.as<int>() + off, nr, 0, stream_), "tile runs");
        hip_check(launch_tile_runs_length(n, src, run_of.as<int>(), run_length_.as<int>() + off, stream_),
                  "tile runs");
        // starts: exclusive scan of the lengths, narrowed into run_start (its
        // last entry, the tile's edge count, is the next tile's first start
        // until that tile writes it)
        hip_check(launch_exclusive_scan_i32(run_length_.as<int>() + off, nr, scan.as<long long>(),
                                            scan_scratch.as<long long>(), stream_),
                  "tile runs");
        hip_check(launch_narrow_offsets(scan.as<long long>(), nr, start, nullptr, stream_), "tile runs");
        hip_check(launch_fill_i32(cursors.as<int>(), nr, 0, stream_), "tile lists");
        hip_check(launch_tile_list_fill(n, src, run_of.as<int>(), start, cursors.as<int>(), tedge_.as<int>() + base,
                                        stream_),
                  "tile lists");
        hip_check(launch_sort_segments(nr, start, tedge_.as<int>() + base, stream_), "tile lists");
    }
    // every tile must have as many runs as its count said
    std::vector<int> seen(tiles, 0);
    if (tiles > 0)
        hip_check(hipMemcpyAsync(seen.data(), counts.as<int>(), tiles * sizeof(int), hipMemcpyDeviceToHost, stream_),
                  "copy");
    wait("tile lists");
    if (seen != tile_runs_) throw std::logic_error("tile run counts of the graph build and the tile lists differ");
}

// Device bytes this evaluator holds for graphs and their work arrays (not
// the model and radial tables).
std::size_t Evaluator::held_graph_bytes() const
{
    const DeviceBuffer* buffers[] = {
        &node_types_, &first_, &receiver_, &source_, &tfirst_, &tedge_, &edge_pair_, &disp_, &positions_,
        &cell_dev_, &xyz_, &r_, &geo_positions_, &geo_edges_, &geo_shifts_, &A0_, &M0_, &H1_, &Phi1_, &A1_,
        &A1adj_, &A0pre_, &direct_, &H1adj_, &msg_, &rpart_, &energies_, &forces_, &atom_forces_, &partials_, &totals_, &scratch_,
        &scale1_, &dot1_, &M0s_, &run_source_, &run_start_, &run_length_, &node_order_, &m0_blocks_, &m0r_blocks_,
        &readout_blocks_, &edge_tiles_, &edge_tiles_l0_, &tile_xyz_, &tile_r_, &tile_pair_, &tile_forces_,
        &pgraph_.first, &pgraph_.sources, &pgraph_.shifts, &pgraph_.fractional_xyz, &pgraph_.fractional_positions};
    std::size_t total = 0;
    for (const DeviceBuffer* b : buffers) total += b->bytes();
    return total;
}

// Device bytes of the graph-wide state of the prepared graph.  Both plans:
// per edge the sources (and for a periodic graph the cell shifts, int8 or
// int32); per node types, receiver offsets, the node order and blocks of
// the node kernels, energies, atom forces, positions and displacements, H1
// and its adjoint and the direct adjoint (periodic: the build's fractional
// positions).  The untiled plan adds per edge the source-major list,
// receivers, pair codes, geometry and directed forces (periodic: fractional
// edge vectors) and per node the source-major offsets; the tiled plan per
// edge the tiles' source-grouped lists (and pair codes when a caller's
// neighbour types differ from its sources') and three ints per run; its
// scalar M0 block shares the direct adjoint's array.
std::size_t Evaluator::graph_bytes_estimate(bool tiled, long long runs) const
{
    const std::size_t N = num_nodes_, E = static_cast<std::size_t>(num_edges_);
    const std::size_t C = C_, f = sizeof(float);
    std::size_t per_edge = sizeof(int);
    std::size_t per_node = 7 * sizeof(int) + 10 * sizeof(double) + (2 * static_cast<std::size_t>(nLM_) + 1) * C * f;
    if (periodic_) {
        per_edge += 3 * static_cast<std::size_t>(pgraph_.shift_bytes);
        per_node += 3 * sizeof(double);
    }
    std::size_t extra = 0;
    if (!tiled) {
        per_edge += 3 * sizeof(int) + 7 * sizeof(double);
        if (periodic_) per_edge += 3 * sizeof(double);
        per_node += sizeof(int);
        // the two edge-tile lists: two ints per tile, at most N + E / 16 tiles
        extra += 4 * sizeof(int) * (N + E / kMinEdgeTile);
    } else {
        per_edge += sizeof(int);
        if (!pair_from_types_) per_edge += sizeof(int);
        extra += 3 * sizeof(int) * static_cast<std::size_t>(std::max(runs, 0LL));
    }
    if (model_.A1_scaled) per_node += 2 * f;
    if (model_.pre_linear_up && !tiled) per_node += C * f;
    return per_edge * E + per_node * N + extra;
}

// Device bytes of the work arrays for `receivers` receivers and `edges`
// edges: A0, A1 and A1_adj [lm], M0 [LM], Phi1 [lme] per receiver and the
// H1-adjoint messages [LM] per edge; the tiled plan's arena also holds each
// tile edge's geometry, pair code and directed force.
std::size_t Evaluator::work_bytes_estimate(long long receivers, long long edges, bool tiled) const
{
    // the unfolded layer-0 path (untiled) keeps the sums before A0_W as well
    const int pre = !tiled && a0_unfold_ ? nlm_ : 0;
    const std::size_t per_node = static_cast<std::size_t>(C_) * sizeof(float) * (3 * nlm_ + pre + nLM_ + nlme_);
    std::size_t per_edge = static_cast<std::size_t>(nLM_) * C_ * sizeof(float);
    if (r1_rev_slices_ > 1) per_edge += 3 * sizeof(double) * r1_rev_slices_;
    if (tiled) per_edge += 7 * sizeof(double) + sizeof(int);
    return per_node * static_cast<std::size_t>(std::max(receivers, 1LL)) +
           per_edge * static_cast<std::size_t>(std::max(edges, 1LL));
}

void Evaluator::set_execution_plan_request(const std::string& algorithm, const std::string& profile,
                                           const std::string& debug_plan)
{
    if (algorithm != "direct")
        throw std::invalid_argument("streamed_edges must be 'direct' on this backend (got '" + algorithm + "').");
    if (profile != "capacity" && profile != "speed")
        throw std::invalid_argument("execution_profile must be 'capacity' or 'speed'.");
    if (!debug_plan.empty() && debug_plan != "mh0-direct-speed" && debug_plan != "mh0-dual-layer-tiled-v1")
        throw std::invalid_argument("_debug_execution_plan must be 'mh0-direct-speed' or 'mh0-dual-layer-tiled-v1' "
                                    "on this backend.");
    if (debug_plan == "mh0-dual-layer-tiled-v1" && profile != "capacity")
        throw std::invalid_argument("MH-0 capacity debug plans require execution_profile='capacity'.");
    invalidate_graph();
    plan_profile_ = profile;
    plan_debug_ = debug_plan;
    plan_report_ = ExecutionPlanReport{};
    plan_report_.requested_profile = profile;
    plan_report_.selection_source = debug_plan.empty() ? "native_request" : "debug_override";
}

namespace {
void json_string(std::string& out, const std::string& v)
{
    out += '"';
    for (char c : v) {
        if (c == '"' || c == '\\') out += '\\';
        out += c;
    }
    out += '"';
}
}  // namespace

std::string ExecutionPlanReport::json() const
{
    std::string out = "{";
    auto key = [&](const char* k) {
        if (out.size() > 1) out += ", ";
        json_string(out, k);
        out += ": ";
    };
    key("requested_algorithm"), json_string(out, requested_algorithm);
    key("requested_profile"), json_string(out, requested_profile);
    key("selection_source"), json_string(out, selection_source);
    key("state"), json_string(out, state);
    key("selected_id"), json_string(out, selected_id);
    key("selection_reason"), json_string(out, selection_reason);
    key("available_bytes"), out += std::to_string(available_bytes);
    key("reserve_bytes"), out += std::to_string(reserve_bytes);
    key("boundary_attempt"), out += boundary_attempt ? "true" : "false";
    key("candidates");
    out += "[";
    for (std::size_t i = 0; i < candidates.size(); ++i) {
        const PlanCandidate& c = candidates[i];
        if (i) out += ", ";
        out += "{\"id\": ";
        json_string(out, c.id);
        out += ", \"qualified\": ";
        out += c.qualified ? "true" : "false";
        out += ", \"estimated_bytes\": " + std::to_string(c.estimated_bytes) + ", \"reason\": ";
        json_string(out, c.reason);
        out += "}";
    }
    out += "]}";
    return out;
}

std::string Evaluator::workspace_json() const
{
    auto sum = [](std::initializer_list<const DeviceBuffer*> buffers) {
        std::size_t total = 0;
        for (const DeviceBuffer* b : buffers) total += b->bytes();
        return total;
    };
    const bool tiled = tile_receivers_ > 0;
    long long max_tile_edges = 0, runs = 0;
    for (int t = 0; tiled && t < num_tiles_; ++t)
        max_tile_edges = std::max(max_tile_edges, tile_first_edge_[t + 1] - tile_first_edge_[t]);
    if (tiled && !tile_run_offsets_.empty()) runs = tile_run_offsets_.back();
    std::size_t free_bytes = 0, total_bytes = 0;
    if (hipMemGetInfo(&free_bytes, &total_bytes) != hipSuccess) free_bytes = total_bytes = 0;
    const std::size_t node_work = sum({&A0_, &A0pre_, &M0_, &M0s_, &Phi1_, &A1_, &A1adj_, &scale1_, &dot1_});
    const std::size_t edge_work = sum({&msg_, &rpart_, &forces_, &tile_forces_, &tile_xyz_, &tile_r_, &tile_pair_});
    std::string out = "{";
    auto field = [&](const char* k, long long v) {
        if (out.size() > 1) out += ", ";
        out += '"';
        out += k;
        out += "\": " + std::to_string(v);
    };
    // 0 when no graph is prepared or a setter has invalidated it
    field("graph_generation", static_cast<long long>(prepared_generation_ == generation_ ? generation_ : 0));
    field("num_nodes", num_nodes_);
    field("num_edges", num_edges_);
    field("tiled", tiled ? 1 : 0);
    field("tile_receivers", tile_receivers_);
    field("num_tiles", tiled ? num_tiles_ : 0);
    field("max_tile_edges", max_tile_edges);
    field("tile_runs", runs);
    field("run_bytes", static_cast<long long>(sum({&run_source_, &run_start_, &run_length_})));
    field("graph_bytes", static_cast<long long>(sum({&node_types_, &first_, &receiver_, &source_, &tfirst_, &tedge_,
                                                     &edge_pair_, &run_source_, &run_start_, &run_length_,
                                                     &node_order_, &m0_blocks_, &m0r_blocks_, &readout_blocks_,
                                                     &pgraph_.first, &pgraph_.sources, &pgraph_.shifts,
                                                     &pgraph_.fractional_xyz, &pgraph_.fractional_positions})));
    field("geometry_bytes", static_cast<long long>(sum({&disp_, &positions_, &cell_dev_, &xyz_, &r_, &geo_positions_,
                                                        &geo_edges_, &geo_shifts_, &tile_xyz_, &tile_r_})));
    field("node_work_bytes", static_cast<long long>(node_work));
    field("edge_work_bytes", static_cast<long long>(edge_work));
    field("phi1_bytes", static_cast<long long>(Phi1_.bytes()));
    field("message_bytes", static_cast<long long>(msg_.bytes()));
    field("readout_bytes", static_cast<long long>(sum({&energies_, &direct_})));
    field("feature_bytes", static_cast<long long>(sum({&H1_, &H1adj_, &atom_forces_})));
    field("reduction_bytes", static_cast<long long>(sum({&partials_, &totals_, &scratch_})));
    field("table_bytes", static_cast<long long>(sum({&type_active_, &r0f_, &r1_, &p0_coef_, &p0_packed_, &p0_offsets_,
                                                     &p1_coef_, &p1_packed_, &p1_offsets_, &h2m0_, &h2m0t_, &e0_,
                                                     &h1w_, &h1wt_, &h2m1_, &h2m1t_, &q_, &w1_, &w2_, &cg_, &p0w_,
                                                     &p0wt_, &residual_, &residual_fused_, &r0u_, &h0s_, &a0w_,
                                                     &a0wt_})));
    field("device_free_bytes", static_cast<long long>(free_bytes));
    field("device_total_bytes", static_cast<long long>(total_bytes));
    field("a0_unfolded", a0_unfold_ ? 1 : 0);
    field("r1_forward_slices", tile_receivers_ > 0 ? r1_slices_ : r1_graph_slices_);
    field("r1_reverse_slices", r1_rev_slices_);
    field("a0_forward_slices", tile_receivers_ > 0 ? 1 : a0_graph_slices_);
    field("edge_tile", num_edge_tiles_ > 0 ? edge_tile_ : 0);
    out += "}";
    return out;
}

// Nodes of each tile (the whole graph untiled) grouped by active type, in
// ascending node order within a type, cut into blocks for the node kernels.
void Evaluator::plan_node_blocks()
{
    const int N = num_nodes_;
    const int tiles = tile_receivers_ > 0 ? num_tiles_ : 1;
    const int T = tile_receivers_ > 0 ? tile_receivers_ : std::max(N, 1);
    const int na = static_cast<int>(active_types_.size());
    std::vector<int> ta(model_.num_elements, -1);
    for (int a = 0; a < na; ++a) ta[active_types_[a]] = a;
    std::vector<int> order;
    order.reserve(N);
    std::vector<NodeBlock> m0b, m0rb, rob;
    // narrower blocks for the two-wave-per-SIMD node kernels (M0 reverse,
    // readout, eight-node M0 forward) of a launch that would otherwise fill
    // the machine less than twice over: more workgroups, fewer registers, a
    // shorter last round
    const long long launch_nodes = std::min(N, T);
    const int block_waves = (C_ + 63) / 64;  // node kernels: one thread per channel
    const long long two_rounds = 2LL * 2 * 4 * std::max(compute_units_, 1);  // waves: 2 per SIMD, 4 SIMDs per CU
    auto narrow = [&](int wide_nodes) {
        return C_ <= 128 && (launch_nodes + wide_nodes - 1) / wide_nodes * block_waves < two_rounds;
    };
    m0r_block_nodes_ = narrow(kM0BlockNodes) ? kM0ReverseBlockNodesNarrow : kM0BlockNodes;
    readout_block_nodes_ = narrow(kReadoutBlockNodes) ? kReadoutBlockNodesNarrow : kReadoutBlockNodes;
    // one node per block where the launch has at most one wave per SIMD:
    // the blocks' serial chains set the time there (medium shape, per call:
    // 135 atoms 255 -> 246 us, 320 atoms 297 -> 292 us; M0 forward and
    // reverse 12 -> 9 us each at 135 atoms, readout 25 -> 23 us; 1,080 atoms
    // 511 -> 526 us).  SXL_NODE_BLOCK=1 / 0 forces the choice (tests).
    bool one_node = launch_nodes * block_waves <= 4LL * std::max(compute_units_, 1);
    if (const char* v = std::getenv("SXL_NODE_BLOCK"); v && v[0]) one_node = v[0] == '1';
    m0_block_nodes_ = narrow(kM0ForwardBlockNodesWide) ? kM0BlockNodes : kM0ForwardBlockNodesWide;
    if (one_node) m0_block_nodes_ = m0r_block_nodes_ = readout_block_nodes_ = 1;
    m0_block_offsets_.assign(tiles + 1, 0);
    m0r_block_offsets_.assign(tiles + 1, 0);
    readout_block_offsets_.assign(tiles + 1, 0);
    std::vector<std::vector<int>> by_type(na);
    type_start_.assign(na, 0);
    type_count_.assign(na, 0);
    for (int t = 0; t < tiles; ++t) {
        const int lo = t * T, hi = std::min(N, lo + T);
        for (auto& v : by_type) v.clear();
        for (int i = lo; i < hi; ++i) by_type[ta[host_types_[i]]].push_back(i);
        for (int a = 0; a < na; ++a) {
            const int start = static_cast<int>(order.size());
            const int n = static_cast<int>(by_type[a].size());
            if (tiles == 1) {
                type_start_[a] = start;
                type_count_[a] = n;
            }
            order.insert(order.end(), by_type[a].begin(), by_type[a].end());
            for (int b = 0; b < n; b += m0_block_nodes_)
                m0b.push_back({start + b, std::min(m0_block_nodes_, n - b), a, 0});
            for (int b = 0; b < n; b += m0r_block_nodes_)
                m0rb.push_back({start + b, std::min(m0r_block_nodes_, n - b), a, 0});
            for (int b = 0; b < n; b += readout_block_nodes_)
                rob.push_back({start + b, std::min(readout_block_nodes_, n - b), a, 0});
        }
        m0_block_offsets_[t + 1] = static_cast<int>(m0b.size());
        m0r_block_offsets_[t + 1] = static_cast<int>(m0rb.size());
        readout_block_offsets_[t + 1] = static_cast<int>(rob.size());
    }
    upload(node_order_, order, stream_, &staged_);
    // untiled plan with at most ten receiver waves per compute unit: the
    // reverse edge kernels, which need no per-receiver reduction, run each
    // receiver's edges in 16-edge tiles, each tile a workgroup of its own
    // (medium shape, per call: 135 atoms 317 -> 266 us, 625 atoms 434 ->
    // 400 us, 1,080 atoms 536 -> 511 us; 1,715 atoms 705 -> 715 us and 5,000
    // atoms 1.64 -> 1.77 ms, where the receivers already fill the machine and
    // each tile repeats its receiver's set-up; 32- and 64-edge tiles gain
    // less at every size).  SXL_EDGE_TILE_LAUNCH=1 / 0 forces the choice and
    // SXL_EDGE_TILE=16 / 32 / 64 the tile (tests).
    num_edge_tiles_ = 0;
    edge_tiles_.release();
    edge_tiles_l0_.release();
    const char* tile_launch = std::getenv("SXL_EDGE_TILE_LAUNCH");
    const long long receiver_waves = static_cast<long long>(N) * ((C_ + 63) / 64);
    const long long cus = std::max(compute_units_, 1);
    const bool edge_tile_launch =
        tile_launch && tile_launch[0] ? tile_launch[0] == '1' : receiver_waves <= 10LL * cus;
    // graphs with at most one receiver wave per SIMD run the second-interaction
    // forward of the (3, 1) and (3, 2) shapes and the layer-0 forward in
    // 64-channel slices whose four waves split each receiver's edges (layer 0,
    // medium shape: 135 atoms 267 -> 252 us per call; 625 atoms 401 -> 403 us,
    // 1,080 atoms 512 -> 520 us when forced).  SXL_A0_FORWARD_SLICES=1 / 0
    // forces the layer-0 choice (tests).
    const bool small_graph = tile_receivers_ == 0 && receiver_waves <= 4LL * cus && (C_ == 128 || C_ == 256);
    r1_graph_slices_ = r1_slices_;
    if (small_graph && model_.l_max == 3 && (model_.L_max == 1 || model_.L_max == 2)) r1_graph_slices_ = C_ / 64;
    bool a0_sliced = small_graph;
    if (const char* t = std::getenv("SXL_A0_FORWARD_SLICES"); t && t[0])
        a0_sliced = t[0] == '1' && tile_receivers_ == 0 && (C_ == 128 || C_ == 256);
    a0_graph_slices_ = a0_sliced ? C_ / 64 : 1;
    edge_tile_ = kMinEdgeTile;
    if (const char* t = std::getenv("SXL_EDGE_TILE"); t && t[0]) {
        const int v = std::atoi(t);
        if (v == 16 || v == 32 || v == 64) edge_tile_ = v;
    }
    if (tile_receivers_ == 0 && N > 0 && edge_tile_launch) {
        std::vector<int> natural, layer0;
        auto add = [&](std::vector<int>& list, int i) {
            for (long long e = host_first_[i]; e < host_first_[i + 1]; e += edge_tile_) {
                list.push_back(i);
                list.push_back(static_cast<int>(e));
            }
        };
        for (int i = 0; i < N; ++i) add(natural, i);
        for (int i : order) add(layer0, i);
        num_edge_tiles_ = static_cast<int>(natural.size() / 2);
        if (num_edge_tiles_ > 0) {
            upload(edge_tiles_, natural, stream_, &staged_);
            upload(edge_tiles_l0_, layer0, stream_, &staged_);
        }
    }
    upload(m0_blocks_, m0b, stream_, &staged_);
    upload(m0r_blocks_, m0rb, stream_, &staged_);
    upload(readout_blocks_, rob, stream_, &staged_);
}

NodeBlocks Evaluator::node_blocks(const DeviceBuffer& blocks, const std::vector<int>& offsets, int tile,
                                  int block_nodes) const
{
    NodeBlocks nb;
    nb.order = node_order_.as<int>();
    nb.blocks = blocks.as<NodeBlock>();
    nb.first = offsets[tile];
    nb.count = offsets[tile + 1] - offsets[tile];
    nb.block_nodes = block_nodes;
    return nb;
}

void Evaluator::invalidate_graph()
{
    wait("synchronize");
    release_replay();
    ++generation_;
    evaluated_generation_ = 0;
    reduced_ = false;
}

void Evaluator::set_allow_fixed_workspace(bool allow)
{
    if (allow == allow_fixed_workspace_) return;
    invalidate_graph();
    allow_fixed_workspace_ = allow;
}

void Evaluator::set_workspace_receiver_limit(int receivers)
{
    if (receivers <= 0) throw std::invalid_argument("Dual-layer workspace receiver limit must be positive.");
    invalidate_graph();
    receiver_limit_ = receivers;
}

// Per-edge state the tiled plan does not keep: released before its edges
// are written, so a capacity graph never holds both.
void Evaluator::release_untiled_edge_state()
{
    wait("synchronize");
    receiver_.release();
    tfirst_.release();
    edge_pair_.release();
    xyz_.release();
    r_.release();
    forces_.release();
    msg_.release();
    rpart_.release();
    pgraph_.fractional_xyz.release();
}

// Pair codes of a caller's graph from its neighbour types (checked against
// the model), and whether they follow from the node types.
std::vector<int> Evaluator::caller_pairs(const int* host_neigh_types, const int* host_sources)
{
    const int N = num_nodes_;
    std::vector<int> host_pairs(static_cast<std::size_t>(num_edges_));
    std::vector<int> ta(model_.num_elements, -1);
    for (std::size_t a = 0; a < active_types_.size(); ++a) ta[active_types_[a]] = static_cast<int>(a);
    const int na = static_cast<int>(active_types_.size());
    pair_from_types_ = true;
    std::size_t e = 0;
    for (int i = 0; i < N; ++i) {
        const int a = ta[host_types_[i]];
        for (long long j = host_first_[i]; j < host_first_[i + 1]; ++j, ++e) {
            const int t = host_neigh_types[e];
            if (t < 0 || t >= model_.num_elements) throw std::out_of_range("MACE radial type index is out of range.");
            const int b = ta[t];
            if (b < 0) throw std::runtime_error("MACE radial cache is not prepared for an active type.");
            if (t != host_types_[host_sources[e]]) pair_from_types_ = false;
            const int po = a * na + b;
            const int pu = shared_pair_tables() ? 0 : a <= b ? a * (2 * na - a - 1) / 2 + b : b * (2 * na - b - 1) / 2 + a;
            host_pairs[e] = po | (pu << 16);
        }
    }
    return host_pairs;
}

// The layer-0 table the selected plan reads on the device, the other one
// released: the folded table for the tiled plan and for the untiled plan with
// few active types, the unfolded table with H0 and A0_W otherwise.
void Evaluator::place_layer0_tables()
{
    if (a0_unfolded()) {
        r0f_.release();
        if (r0u_.bytes() == 0) {
            upload(r0u_, host_r0u_, stream_, &staged_);
            upload(h0s_, host_h0_, stream_, &staged_);
            upload(a0w_, host_a0w_, stream_, &staged_);
            upload(a0wt_, host_a0wt_, stream_, &staged_);
        }
    } else {
        r0u_.release();
        h0s_.release();
        a0w_.release();
        a0wt_.release();
        if (r0f_.bytes() == 0) upload(r0f_, host_r0f_, stream_, &staged_);
    }
}

// Shared tail of both graph preparations, once the plan is selected and the
// sources are on the device.  Untiled: receiver offsets, source-major
// transpose, receivers and pair codes graph-wide.  Tiled: the tile-local
// offsets, source-grouped lists and runs (pair codes are formed per tile,
// or kept graph-wide when a caller's neighbour types differ).  Then the node
// blocks and the work arrays.
void Evaluator::finish_graph(const std::vector<int>& host_pairs)
{
    const int N = num_nodes_;
    const long long E = num_edges_;
    place_layer0_tables();
    if (tile_receivers_ == 0) {
        run_source_.release();
        run_start_.release();
        run_length_.release();
        const int Ei = static_cast<int>(E);  // the untiled plan's edges fit its 32-bit index
        std::vector<int> first(host_first_.begin(), host_first_.end());
        upload(first_, first, stream_, &staged_);
        // transpose: count -> scan -> fill -> sort each source segment ascending
        // (its work arrays live until the preparation's final wait)
        DeviceBuffer counts, offsets64;
        counts.reserve((N + 1) * sizeof(int));
        offsets64.reserve((N + 1) * sizeof(long long));
        scratch_.reserve(scan_scratch_size(N + 1) * sizeof(long long));
        hip_check(hipMemsetAsync(counts.as<void>(), 0, (N + 1) * sizeof(int), stream_), "memset");
        hip_check(launch_transpose_count(Ei, source_.as<int>(), counts.as<int>(), stream_), "transpose");
        hip_check(launch_exclusive_scan_i32(counts.as<int>(), N, offsets64.as<long long>(),
                                            scratch_.as<long long>(), stream_),
                  "scan");
        tfirst_.reserve((N + 1) * sizeof(int));
        hip_check(launch_narrow_offsets(offsets64.as<long long>(), N, tfirst_.as<int>(), nullptr, stream_),
                  "narrow");
        tedge_.reserve(static_cast<std::size_t>(std::max(Ei, 1)) * sizeof(int));
        hip_check(hipMemsetAsync(counts.as<void>(), 0, (N + 1) * sizeof(int), stream_), "memset");
        hip_check(launch_transpose_fill(Ei, source_.as<int>(), tfirst_.as<int>(), counts.as<int>(),
                                        tedge_.as<int>(), stream_),
                  "transpose fill");
        hip_check(launch_sort_segments(N, tfirst_.as<int>(), tedge_.as<int>(), stream_), "sort");
        receiver_.reserve(static_cast<std::size_t>(std::max(Ei, 1)) * sizeof(int));
        hip_check(launch_receivers(N, first_.as<int>(), receiver_.as<int>(), stream_), "receivers");
        if (!host_pairs.empty()) {
            upload(edge_pair_, host_pairs, stream_, &staged_);
        } else {
            edge_pair_.reserve(static_cast<std::size_t>(std::max(Ei, 1)) * sizeof(int));
            hip_check(launch_edge_pairs(Ei, receiver_.as<int>(), source_.as<int>(), node_types_.as<int>(),
                                        type_active_.as<int>(), static_cast<int>(active_types_.size()),
                                        shared_pair_tables(), edge_pair_.as<int>(), stream_),
                      "edge pairs");
        }
    } else {
        if (!pair_from_types_) upload(edge_pair_, host_pairs, stream_, &staged_);
        build_tile_lists();
    }
    plan_node_blocks();
    allocate_workspace();
    wait("graph preparation");
    ++generation_;
    prepared_generation_ = generation_;
    evaluated_generation_ = 0;
    reduced_ = false;
    stats_.graph_builds += 1;
    stats_.last_num_nodes = N;
    stats_.last_num_edges = E;
    stats_.tile_receivers = tile_receivers_;
    stats_.num_tiles = num_tiles_;
}

// Tiles counted for the graph being prepared: only when a tiled plan could
// be chosen (fixed workspace allowed or pinned, more nodes than one tile).
bool Evaluator::tiles_possible(int num_nodes) const
{
    const int T = receiver_limit_ > 0 ? receiver_limit_ : kDefaultTileReceivers;
    return (allow_fixed_workspace_ || plan_debug_ == "mh0-dual-layer-tiled-v1") && num_nodes > T &&
           plan_debug_ != "mh0-direct-speed" && plan_profile_ != "speed";
}

std::uint64_t Evaluator::prepare_graph(int num_nodes, const int* node_types, const int* num_neigh,
                                       const int* neigh_indices, const int* neigh_types)
{
    const CallStart start;
    if (num_nodes < 0 || num_nodes >= std::numeric_limits<int>::max())
        throw std::length_error("MACE graph atom count exceeds the 32-bit CSR limit.");
    std::vector<int> types(node_types, node_types + num_nodes);
    long long E = 0;
    std::vector<long long> first(num_nodes + 1, 0);
    for (int i = 0; i < num_nodes; ++i) {
        if (num_neigh[i] < 0) throw std::invalid_argument("num_neigh must be non-negative.");
        E += num_neigh[i];
        if (E > std::numeric_limits<int>::max())
            throw std::length_error("MACE graph directed-edge count exceeds the 32-bit topology limit.");
        first[i + 1] = E;
    }
    for (long long e = 0; e < E; ++e)
        if (neigh_indices[e] < 0 || neigh_indices[e] >= num_nodes)
            throw std::out_of_range("neighbour index out of range.");
    // from here on the graph state changes: a preparation that fails part way
    // must leave no earlier token valid
    invalidate_graph();
    prepare_active_types(types);
    host_types_ = types;
    num_nodes_ = num_nodes;
    num_edges_ = E;
    periodic_ = false;
    host_first_ = std::move(first);
    upload(node_types_, types, stream_, &staged_);
    std::vector<int> src(neigh_indices, neigh_indices + E);
    upload(source_, src, stream_, &staged_);
    positions_.reserve(static_cast<std::size_t>(std::max(num_nodes, 1)) * 3 * sizeof(double));
    disp_.reserve(static_cast<std::size_t>(std::max(num_nodes, 1)) * 3 * sizeof(double));
    geometry_mode_ = kGeometryNone;
    std::vector<int> pairs = caller_pairs(neigh_types, neigh_indices);
    tile_runs_.clear();
    if (tiles_possible(num_nodes)) count_tile_runs();
    select_plan();
    if (tile_receivers_ > 0) release_untiled_edge_state();
    finish_graph(pairs);
    account_preparation(start);
    return generation_;
}

std::uint64_t Evaluator::prepare_graph_device(int num_nodes, const int* d_node_types, const int* d_num_neigh,
                                              const int* d_neigh_indices, const int* d_neigh_types)
{
    const CallStart start;
    if (num_nodes < 0 || num_nodes >= std::numeric_limits<int>::max())
        throw std::length_error("MACE graph atom count exceeds the 32-bit CSR limit.");
    // the per-node arrays come to the host (active types, node blocks, plan)
    std::vector<int> types(num_nodes), counts(num_nodes);
    if (num_nodes > 0) {
        hip_check(hipMemcpyAsync(types.data(), d_node_types, num_nodes * sizeof(int), hipMemcpyDeviceToHost, stream_),
                  "node types");
        hip_check(hipMemcpyAsync(counts.data(), d_num_neigh, num_nodes * sizeof(int), hipMemcpyDeviceToHost, stream_),
                  "num_neigh");
    }
    wait("graph arrays");
    long long E = 0;
    std::vector<long long> first(num_nodes + 1, 0);
    for (int i = 0; i < num_nodes; ++i) {
        if (counts[i] < 0) throw std::invalid_argument("num_neigh must be non-negative.");
        E += counts[i];
        if (E > std::numeric_limits<int>::max())
            throw std::length_error("MACE graph directed-edge count exceeds the 32-bit topology limit.");
        first[i + 1] = E;
    }
    for (int t : types)
        if (t < 0 || t >= model_.num_elements) throw std::out_of_range("MACE radial type index is out of range.");
    invalidate_graph();
    prepare_active_types(types);
    host_types_ = types;
    num_nodes_ = num_nodes;
    num_edges_ = E;
    periodic_ = false;
    host_first_ = std::move(first);
    upload(node_types_, types, stream_, &staged_);
    source_.reserve(static_cast<std::size_t>(std::max<long long>(E, 1)) * sizeof(int));
    if (E > 0)
        hip_check(hipMemcpyAsync(source_.as<int>(), d_neigh_indices, static_cast<std::size_t>(E) * sizeof(int),
                                 hipMemcpyDeviceToDevice, stream_),
                  "neighbour indices");
    // neighbour indices and types checked on the device: out-of-range index,
    // out-of-range type, inactive type, type differing from the source's
    DeviceBuffer flags;
    flags.reserve(4 * sizeof(unsigned long long));
    hip_check(hipMemsetAsync(flags.as<void>(), 0, 4 * sizeof(unsigned long long), stream_), "memset");
    hip_check(launch_check_neighbors(E, num_nodes, source_.as<int>(), d_neigh_types, node_types_.as<int>(),
                                     type_active_.as<int>(), model_.num_elements, flags.as<unsigned long long>(),
                                     stream_),
              "neighbour check");
    unsigned long long bad[4] = {};
    hip_check(hipMemcpyAsync(bad, flags.as<void>(), sizeof(bad), hipMemcpyDeviceToHost, stream_), "copy");
    wait("neighbour check");
    if (bad[0]) throw std::out_of_range("neighbour index out of range.");
    if (bad[1]) throw std::out_of_range("MACE radial type index is out of range.");
    if (bad[2]) throw std::runtime_error("MACE radial cache is not prepared for an active type.");
    positions_.reserve(static_cast<std::size_t>(std::max(num_nodes, 1)) * 3 * sizeof(double));
    disp_.reserve(static_cast<std::size_t>(std::max(num_nodes, 1)) * 3 * sizeof(double));
    geometry_mode_ = kGeometryNone;
    std::vector<int> pairs;
    pair_from_types_ = true;
    if (bad[3]) {
        // neighbour types that differ from their sources': pair codes on the host
        std::vector<int> src(static_cast<std::size_t>(E)), ntypes(static_cast<std::size_t>(E));
        hip_check(hipMemcpyAsync(src.data(), source_.as<int>(), E * sizeof(int), hipMemcpyDeviceToHost, stream_),
                  "copy");
        hip_check(hipMemcpyAsync(ntypes.data(), d_neigh_types, E * sizeof(int), hipMemcpyDeviceToHost, stream_),
                  "copy");
        wait("neighbour types");
        pairs = caller_pairs(ntypes.data(), src.data());
    }
    tile_runs_.clear();
    if (tiles_possible(num_nodes)) count_tile_runs();
    select_plan();
    if (tile_receivers_ > 0) release_untiled_edge_state();
    finish_graph(pairs);
    account_preparation(start);
    return generation_;
}

void validate_periodic_inputs(int num_nodes, const double* cell, const double* inverse_cell, double cutoff)
{
    if (!std::isfinite(cutoff) || !(cutoff > 0.0))
        throw std::invalid_argument("neighbor graph cutoff must be finite and positive");
    if (num_nodes < 0 || num_nodes >= std::numeric_limits<int>::max())
        throw std::length_error("neighbor graph exceeds 32-bit node indexing");
    for (int i = 0; i < 9; ++i)
        if (!std::isfinite(cell[i]) || !std::isfinite(inverse_cell[i]))
            throw std::invalid_argument("neighbor graph cell must be finite");
    for (int row = 0; row < 3; ++row)
        for (int column = 0; column < 3; ++column) {
            double product = 0.0;
            for (int inner = 0; inner < 3; ++inner) product += cell[3 * row + inner] * inverse_cell[3 * inner + column];
            if (std::abs(product - (row == column ? 1.0 : 0.0)) > 1e-9)
                throw std::invalid_argument("neighbor graph cell and inverse cell are inconsistent");
        }
}

NeighborPlan neighbor_plan(int num_nodes, const double* cell, const double* inverse_cell, double cutoff)
{
    validate_periodic_inputs(num_nodes, cell, inverse_cell, cutoff);
    NeighborPlan plan;
    const int N = num_nodes;
    plan.num_nodes = N;
    std::memcpy(plan.cell, cell, sizeof(plan.cell));
    std::memcpy(plan.inverse_cell, inverse_cell, sizeof(plan.inverse_cell));
    plan.cutoff_squared = cutoff * cutoff;
    for (int axis = 0; axis < 3; ++axis) {
        double inverse_norm_squared = 0.0;
        for (int component = 0; component < 3; ++component) {
            const double v = inverse_cell[3 * component + axis];
            inverse_norm_squared += v * v;
        }
        if (!(inverse_norm_squared > 0.0)) throw std::invalid_argument("neighbor graph cell must be invertible");
        const double face_height = 1.0 / std::sqrt(inverse_norm_squared);
        const double bins = std::floor(face_height / cutoff);
        if (bins >= static_cast<double>(std::numeric_limits<int>::max()))
            throw std::length_error("neighbor graph bin extent exceeds 32-bit indexing");
        plan.bins[axis] = std::max(1, static_cast<int>(bins));
        const double reach = std::ceil(cutoff * std::sqrt(inverse_norm_squared) * plan.bins[axis]) + 1.0;
        if (reach >= static_cast<double>(std::numeric_limits<int>::max() / 2))
            throw std::length_error("neighbor graph stencil exceeds 32-bit indexing");
        plan.reach[axis] = std::max(1, static_cast<int>(reach));
    }
    const std::size_t num_bins_size =
        static_cast<std::size_t>(plan.bins[0]) * plan.bins[1] * static_cast<std::size_t>(plan.bins[2]);
    if (num_bins_size >= static_cast<std::size_t>(std::numeric_limits<int>::max()))
        throw std::length_error("neighbor graph bin count exceeds 32-bit indexing");
    return plan;
}

int neighbor_plan_bins(const NeighborPlan& plan) { return plan.bins[0] * plan.bins[1] * plan.bins[2]; }

void count_periodic_graph(const double* d_positions, int num_nodes, const double* cell, const double* inverse_cell,
                          double cutoff, hipStream_t stream, DeviceBuffer& fractional_positions, PeriodicCount& c,
                          int tile_receivers)
{
    c.plan = neighbor_plan(num_nodes, cell, inverse_cell, cutoff);
    const NeighborPlan& plan = c.plan;
    const int N = num_nodes;
    const int num_bins = neighbor_plan_bins(plan);
    DeviceBuffer bin_sizes, bin_off64, counts, scratch, small, last_tile;
    const std::size_t N3 = static_cast<std::size_t>(std::max(N, 1)) * 3;
    fractional_positions.reserve(N3 * sizeof(double));
    c.wp.reserve(N3 * sizeof(double));
    c.wf.reserve(N3 * sizeof(double));
    c.wrap.reserve(N3 * sizeof(int));
    c.atom_bins.reserve(std::max(N, 1) * sizeof(int));
    bin_sizes.reserve((num_bins + 1) * sizeof(int));
    bin_off64.reserve((num_bins + 1) * sizeof(long long));
    c.bin_offsets.reserve((num_bins + 1) * sizeof(int));
    c.bin_atoms.reserve(std::max(N, 1) * sizeof(int));
    counts.reserve(std::max(N, 1) * sizeof(long long));
    c.offsets.reserve((static_cast<std::size_t>(N) + 1) * sizeof(long long));
    scratch.reserve(scan_scratch_size(std::max(num_bins, N) + 1) * sizeof(long long));
    const int tiles = tile_receivers > 0 && N > 0 ? static_cast<int>((static_cast<long long>(N) + tile_receivers - 1) /
                                                                     tile_receivers)
                                                  : 0;
    // small: [0] largest shift component, [1..tiles] distinct sources per tile
    small.reserve((1 + static_cast<std::size_t>(tiles)) * sizeof(int));
    hip_check(launch_fill_i32(small.as<int>(), 1 + tiles, 0, stream), "clear");
    hip_check(hipMemsetAsync(bin_sizes.as<void>(), 0, (num_bins + 1) * sizeof(int), stream), "memset");
    hip_check(launch_neighbor_bins(plan, d_positions, fractional_positions.as<double>(), c.wp.as<double>(),
                                   c.wf.as<double>(), c.wrap.as<int>(), c.atom_bins.as<int>(), bin_sizes.as<int>(),
                                   stream),
              "bins");
    hip_check(launch_exclusive_scan_i32(bin_sizes.as<int>(), num_bins, bin_off64.as<long long>(),
                                        scratch.as<long long>(), stream),
              "bin scan");
    hip_check(launch_narrow_offsets(bin_off64.as<long long>(), num_bins, c.bin_offsets.as<int>(), nullptr, stream),
              "narrow");
    // cursors start at the bin offsets
    hip_check(hipMemcpyAsync(bin_sizes.as<int>(), c.bin_offsets.as<int>(), num_bins * sizeof(int),
                             hipMemcpyDeviceToDevice, stream),
              "cursors");
    hip_check(launch_neighbor_fill_bins(plan, c.atom_bins.as<int>(), c.bin_offsets.as<int>(), bin_sizes.as<int>(),
                                        c.bin_atoms.as<int>(), stream),
              "fill bins");
    hip_check(launch_sort_segments(num_bins, c.bin_offsets.as<int>(), c.bin_atoms.as<int>(), stream), "sort bins");
    EdgeOutputs o;
    o.counts = counts.as<long long>();
    o.max_shift = small.as<int>();
    if (tiles > 0) {
        // receiver tiles in order, each marking the sources it has seen
        last_tile.reserve(std::max(N, 1) * sizeof(int));
        hip_check(launch_fill_i32(last_tile.as<int>(), N, -1, stream), "clear");
        o.last_tile = last_tile.as<int>();
        for (int t = 0; t < tiles; ++t) {
            o.tile = t;
            o.tile_runs = small.as<int>() + 1 + t;
            const int begin = t * tile_receivers;
            hip_check(launch_neighbor_edges(plan, c.wp.as<double>(), c.wf.as<double>(), c.wrap.as<int>(),
                                            c.atom_bins.as<int>(), c.bin_offsets.as<int>(), c.bin_atoms.as<int>(),
                                            begin, std::min(tile_receivers, N - begin), o, stream),
                      "count edges");
        }
    } else {
        hip_check(launch_neighbor_edges(plan, c.wp.as<double>(), c.wf.as<double>(), c.wrap.as<int>(),
                                        c.atom_bins.as<int>(), c.bin_offsets.as<int>(), c.bin_atoms.as<int>(), 0, N,
                                        o, stream),
                  "count edges");
    }
    hip_check(launch_exclusive_scan_i64(counts.as<long long>(), N, c.offsets.as<long long>(), scratch.as<long long>(),
                                        stream),
              "edge scan");
    c.host_first.resize(static_cast<std::size_t>(N) + 1);
    hip_check(hipMemcpyAsync(c.host_first.data(), c.offsets.as<long long>(), (N + 1) * sizeof(long long),
                             hipMemcpyDeviceToHost, stream),
              "offsets copy");
    std::vector<int> small_host(1 + tiles);
    hip_check(hipMemcpyAsync(small_host.data(), small.as<int>(), (1 + tiles) * sizeof(int), hipMemcpyDeviceToHost,
                             stream),
              "copy");
    hip_check(host_fence(stream), "edge count");
    c.num_edges = c.host_first[N];
    c.max_shift = small_host[0];
    c.tile_receivers = tiles > 0 ? tile_receivers : 0;
    c.tile_runs.assign(small_host.begin() + 1, small_host.end());
}

void fill_periodic_graph(const PeriodicCount& c, hipStream_t stream, int* sources, int* shifts, signed char* shifts8,
                         double* fractional_xyz)
{
    EdgeOutputs o;
    o.offsets = c.offsets.as<long long>();
    o.sources = sources;
    o.shifts = shifts;
    o.shifts8 = shifts8;
    o.frac = fractional_xyz;
    hip_check(launch_neighbor_edges(c.plan, c.wp.as<double>(), c.wf.as<double>(), c.wrap.as<int>(),
                                    c.atom_bins.as<int>(), c.bin_offsets.as<int>(), c.bin_atoms.as<int>(), 0,
                                    c.plan.num_nodes, o, stream),
              "fill edges");
}

void build_periodic_graph(const double* d_positions, int num_nodes, const double* cell, const double* inverse_cell,
                          double cutoff, hipStream_t stream, PeriodicGraph& out)
{
    PeriodicCount c;
    count_periodic_graph(d_positions, num_nodes, cell, inverse_cell, cutoff, stream, out.fractional_positions, c, 0);
    if (c.num_edges > std::numeric_limits<int>::max())
        throw std::length_error("neighbor graph exceeds 32-bit edge indexing");
    const int N = num_nodes;
    const std::size_t E = static_cast<std::size_t>(std::max<long long>(c.num_edges, 1));
    out.first.reserve((N + 1) * sizeof(int));
    hip_check(launch_narrow_offsets(c.offsets.as<long long>(), N, out.first.as<int>(), nullptr, stream), "narrow");
    out.sources.reserve(E * sizeof(int));
    // sizes in size_t: 3 E overflows 32 bits beyond ~1.43 G edges
    out.shifts.reserve(E * 3 * sizeof(int));
    out.shift_bytes = 4;
    out.fractional_xyz.reserve(E * 3 * sizeof(double));
    fill_periodic_graph(c, stream, out.sources.as<int>(), out.shifts.as<int>(), nullptr,
                        out.fractional_xyz.as<double>());
    hip_check(host_fence(stream), "graph build");
    out.num_nodes = N;
    out.num_edges = c.num_edges;
}

std::uint64_t Evaluator::prepare_periodic_graph(int num_nodes, const int* node_types, const double* positions,
                                                bool device_positions, const double* cell,
                                                const double* inverse_cell, double cutoff)
{
    const CallStart start;
    validate_periodic_inputs(num_nodes, cell, inverse_cell, cutoff);
    std::vector<int> types(node_types, node_types + num_nodes);
    // from here on the graph state changes: a preparation that fails part way
    // must leave no earlier token valid
    invalidate_graph();
    prepare_active_types(types);
    const int N = num_nodes;
    positions_.reserve(static_cast<std::size_t>(std::max(N, 1)) * 3 * sizeof(double));
    if (N > 0)
        hip_check(hipMemcpyAsync(positions_.as<double>(), positions, N * 3 * sizeof(double),
                                 device_positions ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, stream_),
                  "positions");
    disp_.reserve(static_cast<std::size_t>(std::max(N, 1)) * 3 * sizeof(double));
    // count pass (with the distinct sources per tile when a tiled plan could
    // be chosen), then the plan, then the edges it needs
    auto count = std::make_unique<PeriodicCount>();
    const int T = receiver_limit_ > 0 ? receiver_limit_ : kDefaultTileReceivers;
    count_periodic_graph(positions_.as<double>(), N, cell, inverse_cell, cutoff, stream_,
                         pgraph_.fractional_positions, *count, tiles_possible(N) ? T : 0);
    host_types_ = types;
    num_nodes_ = N;
    num_edges_ = count->num_edges;
    host_first_ = std::move(count->host_first);
    tile_runs_ = count->tile_runs;
    periodic_ = true;
    pair_from_types_ = true;
    pgraph_.shift_bytes = count->max_shift <= 127 ? 1 : 4;
    std::memcpy(cell_, cell, sizeof(cell_));
    std::memcpy(inverse_cell_, inverse_cell, sizeof(inverse_cell_));
    select_plan();
    const bool tiled = tile_receivers_ > 0;
    if (tiled) release_untiled_edge_state();
    const std::size_t E = static_cast<std::size_t>(std::max<long long>(num_edges_, 1));
    source_.reserve(E * sizeof(int));
    pgraph_.shifts.reserve(E * 3 * static_cast<std::size_t>(pgraph_.shift_bytes));
    // the untiled plan forms edge vectors from the build's fractional ones;
    // the tiled plan forms them per tile from the shifts (bit for bit)
    if (!tiled) pgraph_.fractional_xyz.reserve(E * 3 * sizeof(double));
    fill_periodic_graph(*count, stream_, source_.as<int>(), pgraph_.shift_bytes == 4 ? pgraph_.shifts.as<int>() : nullptr,
                        pgraph_.shift_bytes == 1 ? pgraph_.shifts.as<signed char>() : nullptr,
                        tiled ? nullptr : pgraph_.fractional_xyz.as<double>());
    pgraph_.first.release();
    pgraph_.sources.release();
    pgraph_.num_nodes = N;
    pgraph_.num_edges = num_edges_;
    upload(node_types_, types, stream_, &staged_);
    upload_cell();
    finish_graph({});
    count.reset();  // the count's work arrays (finish_graph has waited for the fill)
    // the build's fractional positions and edge vectors are the graph's geometry
    geometry_mode_ = kGeometryBuilt;
    geometry_generation_ = generation_;
    geometry_pbc_ = 7;
    account_preparation(start);
    return generation_;
}

void Evaluator::upload_cell()
{
    std::vector<double> cellv(cell_, cell_ + 9);
    cellv.insert(cellv.end(), inverse_cell_, inverse_cell_ + 9);
    upload(cell_dev_, cellv, stream_, &staged_);
}

// New cell for the prepared graph (reference update_factorized_cell): edge
// vectors are formed from the build's fractional edge vectors in this cell
// plus the atoms' minimum-image displacements, so a strained or sheared cell
// reuses the graph while it still covers the cutoff.
void Evaluator::set_cell(const double* cell, const double* inverse_cell)
{
    release_replay();  // the captured totals kernel holds the old volume
    std::memcpy(cell_, cell, sizeof(cell_));
    std::memcpy(inverse_cell_, inverse_cell, sizeof(inverse_cell_));
    upload_cell();
}

namespace {
double determinant3(const double* c)
{
    return c[0] * (c[4] * c[8] - c[5] * c[7]) - c[1] * (c[3] * c[8] - c[5] * c[6]) +
           c[2] * (c[3] * c[7] - c[4] * c[6]);
}

bool all_finite(const double* p, std::size_t n)
{
    for (std::size_t i = 0; i < n; ++i)
        if (!std::isfinite(p[i])) return false;
    return true;
}
}  // namespace

// Requires fractional geometry (the device-built graph's, or the caller's) or
// shift geometry (reference update_factorized_cell,
// mace_kokkos_factorized_lifecycle.cpp:2735-2780).
void Evaluator::update_cell(std::uint64_t generation, const double* cell, const double* inverse_cell)
{
    check_generation(generation);
    if (geometry_generation_ != generation_ ||
        (geometry_mode_ != kGeometryBuilt && geometry_mode_ != kGeometryFractional &&
         geometry_mode_ != kGeometryShifts))
        throw std::invalid_argument(
            "Prepared Execution R1 cell update requires current graph and fractional or shift geometry tokens.");
    if (geometry_mode_ == kGeometryBuilt) {
        validate_periodic_inputs(num_nodes_, cell, inverse_cell, 1.0);
    } else {
        if (!all_finite(cell, 9) || !all_finite(inverse_cell, 9))
            throw std::invalid_argument("Prepared Execution R1 cell matrices contain a non-finite value.");
        const double det = determinant3(cell);
        if (!std::isfinite(det) || det == 0.0)
            throw std::invalid_argument("Prepared Execution R1 cell matrix must be invertible.");
    }
    set_cell(cell, inverse_cell);
}

// Caller geometry of a prepared graph (reference prepare_factorized_geometry
// and prepare_factorized_fractional_geometry,
// mace_kokkos_factorized_lifecycle.cpp:2455-2568, 2699-2733): same checks and
// messages; the arrays are copied to the device.
void Evaluator::prepare_geometry(std::uint64_t generation, const double* reference_positions,
                                 std::size_t num_positions, const double* reference_xyz, std::size_t num_xyz,
                                 const double* cell, const double* inverse_cell, const int* pbc, bool fractional)
{
    release_replay();  // the captured geometry kernels hold the old reference geometry
    if (fractional) {
        if (!(pbc[0] && pbc[1] && pbc[2]))
            throw std::invalid_argument("Fractional Execution R1 geometry requires a fully periodic cell.");
        const double det = determinant3(cell);
        if (!std::isfinite(det) || det == 0.0)
            throw std::invalid_argument("Fractional Execution R1 cell matrix must be invertible.");
    }
    if (generation == 0 || generation != generation_)
        throw std::invalid_argument("Execution R1 geometry requires the current prepared graph token.");
    const std::size_t N = num_nodes_, E = static_cast<std::size_t>(num_edges_);
    if (num_positions != 3 * N || num_xyz != 3 * E)
        throw std::invalid_argument("Execution R1 prepared geometry extents are inconsistent.");
    if (!all_finite(reference_positions, num_positions) || !all_finite(reference_xyz, num_xyz) ||
        !all_finite(cell, 9) || !all_finite(inverse_cell, 9))
        throw std::invalid_argument("Execution R1 prepared geometry contains a non-finite value.");
    geometry_mode_ = kGeometryNone;
    upload(geo_positions_, std::vector<double>(reference_positions, reference_positions + num_positions), stream_, &staged_);
    upload(geo_edges_, std::vector<double>(reference_xyz, reference_xyz + num_xyz), stream_, &staged_);
    set_cell(cell, inverse_cell);
    geometry_pbc_ = (pbc[0] ? 1 : 0) | (pbc[1] ? 2 : 0) | (pbc[2] ? 4 : 0);
    geometry_mode_ = fractional ? kGeometryFractional : kGeometryCartesian;
    geometry_generation_ = generation_;
}

// Positions plus integer cell shifts per edge (reference
// prepare_factorized_shift_geometry, mace_kokkos_factorized_lifecycle.cpp:2570-2697):
// 12 bytes per edge instead of 24.  The reference accepts it only for its
// tiled plans; here both plans form edge vectors from it.
void Evaluator::prepare_shift_geometry(std::uint64_t generation, const double* reference_positions,
                                       std::size_t num_positions, const int* shifts, std::size_t num_shifts,
                                       const double* cell, const double* inverse_cell, const int* pbc)
{
    release_replay();  // the captured geometry kernels hold the old reference geometry
    if (generation == 0 || generation != generation_)
        throw std::invalid_argument("Shift geometry requires the current prepared graph token.");
    const std::size_t N = num_nodes_, E = static_cast<std::size_t>(num_edges_);
    if (num_positions != 3 * N || num_shifts != 3 * E)
        throw std::invalid_argument("Shift geometry extents are inconsistent.");
    if (!all_finite(reference_positions, num_positions) || !all_finite(cell, 9) || !all_finite(inverse_cell, 9))
        throw std::invalid_argument("Shift geometry contains a non-finite value.");
    geometry_mode_ = kGeometryNone;
    upload(geo_positions_, std::vector<double>(reference_positions, reference_positions + num_positions), stream_, &staged_);
    upload(geo_shifts_, std::vector<int>(shifts, shifts + num_shifts), stream_, &staged_);
    set_cell(cell, inverse_cell);
    geometry_pbc_ = (pbc[0] ? 1 : 0) | (pbc[1] ? 2 : 0) | (pbc[2] ? 4 : 0);
    geometry_mode_ = kGeometryShifts;
    geometry_generation_ = generation_;
}

void Evaluator::validate_graph_cardinality(std::uint64_t num_receivers, std::uint64_t num_feature_nodes,
                                           std::uint64_t num_edges) const
{
    constexpr std::uint64_t int_max = static_cast<std::uint64_t>(std::numeric_limits<int>::max());
    if (num_receivers >= int_max)
        throw std::length_error("MACE graph atom count " + std::to_string(num_receivers) +
                                " exceeds the 32-bit CSR limit " + std::to_string(int_max - 1) + ".");
    if (num_feature_nodes >= int_max)
        throw std::length_error("MACE graph feature-node count " + std::to_string(num_feature_nodes) +
                                " exceeds the 32-bit CSR limit " + std::to_string(int_max - 1) + ".");
    if (num_feature_nodes < num_receivers)
        throw std::invalid_argument("MACE graph feature-node count is smaller than its receiver count.");
    if (num_edges > int_max)
        throw std::length_error("MACE graph directed-edge count " + std::to_string(num_edges) +
                                " exceeds the 32-bit topology limit " + std::to_string(int_max) + ".");
}

GeometryRef Evaluator::geometry_ref() const
{
    GeometryRef g;
    if (geometry_mode_ == kGeometryBuilt) {
        // the build's fractional positions with its fractional edge vectors,
        // or (tiled plan, which does not keep those) with its cell shifts,
        // from which the same vectors are formed
        g.positions = pgraph_.fractional_positions.as<double>();
        if (pgraph_.fractional_xyz.bytes() > 0) {
            g.edges = pgraph_.fractional_xyz.as<double>();
        } else if (pgraph_.shift_bytes == 1) {
            g.shifts8 = pgraph_.shifts.as<signed char>();
        } else {
            g.shifts = pgraph_.shifts.as<int>();
        }
        g.fractional = 1;
        g.built = 1;
        g.pbc = 7;
        return g;
    }
    g.positions = geo_positions_.as<double>();
    if (geometry_mode_ == kGeometryShifts)
        g.shifts = geo_shifts_.as<int>();
    else
        g.edges = geo_edges_.as<double>();
    g.fractional = geometry_mode_ == kGeometryFractional ? 1 : 0;
    g.pbc = geometry_pbc_;
    return g;
}

void Evaluator::require_geometry(std::uint64_t generation) const
{
    check_generation(generation);
    if (geometry_mode_ == kGeometryNone || geometry_generation_ != generation_)
        throw std::invalid_argument("Execution R1 positions require current graph and geometry tokens.");
}

void Evaluator::graph_arrays(std::uint64_t generation, int* num_neigh, int* receiver_offsets, int* sources,
                             int* shifts, double* fractional_xyz) const
{
    check_generation(generation);
    const int N = num_nodes_;
    const long long E = num_edges_;
    // the arrays are int32 CSR: as the reference, graphs beyond it are not
    // exported (symmetrix/source/symmetrix/calculator.py:88-104)
    if (E > edge_index_limit_)
        throw std::length_error("MACE graph directed-edge count exceeds the 32-bit topology limit.");
    const std::size_t En = static_cast<std::size_t>(E);
    if (sources && E)
        hip_check(hipMemcpyAsync(sources, source_.as<int>(), En * sizeof(int), hipMemcpyDeviceToHost, stream_), "copy");
    std::vector<int> sh;
    std::vector<int> src;
    std::vector<double> frac;
    const bool rebuild_frac = periodic_ && fractional_xyz && E && pgraph_.fractional_xyz.bytes() == 0;
    if (periodic_ && E && (shifts || rebuild_frac)) {
        if (pgraph_.shift_bytes == 1) {
            std::vector<signed char> s8(3 * En);
            hip_check(hipMemcpyAsync(s8.data(), pgraph_.shifts.as<signed char>(), 3 * En, hipMemcpyDeviceToHost,
                                     stream_),
                      "copy");
            hip_check(host_fence(stream_), "graph copy");
            sh.assign(s8.begin(), s8.end());
        } else {
            sh.resize(3 * En);
            hip_check(hipMemcpyAsync(sh.data(), pgraph_.shifts.as<int>(), 3 * En * sizeof(int),
                                     hipMemcpyDeviceToHost, stream_),
                      "copy");
        }
    }
    if (periodic_ && fractional_xyz && E && !rebuild_frac)
        hip_check(hipMemcpyAsync(fractional_xyz, pgraph_.fractional_xyz.as<double>(), 3 * En * sizeof(double),
                                 hipMemcpyDeviceToHost, stream_),
                  "copy");
    if (rebuild_frac) {
        src.resize(En);
        frac.resize(3 * static_cast<std::size_t>(N));
        hip_check(hipMemcpyAsync(src.data(), source_.as<int>(), En * sizeof(int), hipMemcpyDeviceToHost, stream_),
                  "copy");
        hip_check(hipMemcpyAsync(frac.data(), pgraph_.fractional_positions.as<double>(), N * 3 * sizeof(double),
                                 hipMemcpyDeviceToHost, stream_),
                  "copy");
    }
    hip_check(host_fence(stream_), "graph copy");
    if (receiver_offsets)
        for (int i = 0; i <= N; ++i) receiver_offsets[i] = static_cast<int>(host_first_[i]);
    if (num_neigh)
        for (int i = 0; i < N; ++i) num_neigh[i] = static_cast<int>(host_first_[i + 1] - host_first_[i]);
    if (shifts && periodic_ && E) std::copy(sh.begin(), sh.end(), shifts);
    if (rebuild_frac) {
        // the tiled plan keeps the cell shifts only: the fractional edge
        // vector is formed as the build formed it (positions wrapped to
        // [0, 1), their difference, plus the image), so it equals the
        // build's value bit for bit
        for (int i = 0; i < N; ++i)
            for (long long e = host_first_[i]; e < host_first_[i + 1]; ++e)
                for (int a = 0; a < 3; ++a) {
                    const double pj = frac[3 * static_cast<std::size_t>(src[e]) + a];
                    const double pi = frac[3 * static_cast<std::size_t>(i) + a];
                    const double fj = std::floor(pj), fi = std::floor(pi);
                    const int image = sh[3 * e + a] + static_cast<int>(fj) - static_cast<int>(fi);
                    fractional_xyz[3 * e + a] = ((pj - fj) - (pi - fi)) + static_cast<double>(image);
                }
    }
}

void Evaluator::enqueue_positions(const double* src, bool device_positions)
{
    const int N = num_nodes_;
    if (N > 0 && !device_positions)
        hip_check(hipMemcpyAsync(positions_.as<double>(), pinned_positions_.as<double>(),
                                 static_cast<std::size_t>(N) * 3 * sizeof(double), hipMemcpyHostToDevice, stream_),
                  "positions");
    mark(kStageGeometry, false);
    const double* cell = cell_dev_.as<double>();
    const GeometryRef ref = geometry_ref();
    hip_check(launch_atom_displacements(N, src, ref, cell, cell + 9, disp_.as<double>(), totals_.as<double>() + 12,
                                        stream_),
              "displacements");
    // the tiled plan forms each tile's edges from the displacements per tile
    if (tile_receivers_ == 0)
        hip_check(launch_edge_geometry(static_cast<int>(num_edges_), receiver_.as<int>(), source_.as<int>(), ref,
                                       disp_.as<double>(), cell, model_.r_cut, xyz_.as<double>(), r_.as<double>(),
                                       reinterpret_cast<unsigned long long*>(totals_.as<double>() + 13), stream_),
                  "edge geometry");
    mark(kStageGeometry, true);
}

bool Evaluator::ReplayKey::operator==(const ReplayKey& o) const
{
    if (generation != o.generation || positions != o.positions || device != o.device) return false;
    for (int q = 0; q < 9; ++q)
        if (cell[q] != o.cell[q]) return false;
    return true;
}

void Evaluator::release_replay()
{
    if (replay_exec_) (void)hipGraphExecDestroy(replay_exec_);
    if (replay_graph_) (void)hipGraphDestroy(replay_graph_);
    replay_exec_ = nullptr;
    replay_graph_ = nullptr;
    replay_key_ = ReplayKey{};
    replay_launches_ = 0;
}

void Evaluator::set_graph_replay(bool enable)
{
    if (!enable) release_replay();
    graph_replay_ = enable;
}

void Evaluator::compute_positions(std::uint64_t generation, const double* positions, bool device_positions)
{
    const CallStart start;
    require_geometry(generation);
    const int N = num_nodes_;
    // device positions are read in place by the displacement kernel (nothing
    // later in the evaluation reads them); host positions are staged through
    // pinned memory, whose copy is DMA queued with the kernels (the previous
    // evaluation's wait has drained the buffer)
    const double* src = device_positions ? positions : positions_.as<double>();
    if (N > 0 && !device_positions) {
        const std::size_t bytes = static_cast<std::size_t>(N) * 3 * sizeof(double);
        pinned_positions_.reserve(bytes);
        std::memcpy(pinned_positions_.as<double>(), positions, bytes);
    }
    results_to_host_ = !device_positions;
    for (int i = 0; i < kNumStages; ++i) stage_used_[i] = false;
    check_geometry_ = true;
    explicit_geometry_ = false;
    if (graph_replay_ && tile_receivers_ == 0 && !profiling_ && N > 0) {
        const auto t0 = std::chrono::steady_clock::now();
        ReplayKey key;
        key.generation = generation_;
        key.positions = device_positions ? positions : pinned_positions_.as<double>();
        key.device = device_positions;
        std::copy(cell_, cell_ + 9, key.cell);
        if (!replay_exec_ || !(key == replay_key_)) {
            release_replay();
            const std::uint64_t before = thread_counters().launches;
            hip_check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "graph capture");
            hipGraph_t graph = nullptr;
            try {
                enqueue_positions(src, device_positions);
                enqueue_evaluation();
                enqueue_totals();
            } catch (...) {
                (void)hipStreamEndCapture(stream_, &graph);
                if (graph) (void)hipGraphDestroy(graph);
                (void)hipGetLastError();
                throw;
            }
            hip_check(hipStreamEndCapture(stream_, &graph), "graph capture");
            replay_graph_ = graph;
            hip_check(hipGraphInstantiate(&replay_exec_, replay_graph_, nullptr, nullptr, 0), "graph instantiate");
            replay_key_ = key;
            // the captured launches ran no kernel: counted at each replay
            replay_launches_ = static_cast<long long>(thread_counters().launches - before);
            thread_counters().launches = before;
        }
        hip_check(hipGraphLaunch(replay_exec_, stream_), "graph launch");
        thread_counters().launches += static_cast<std::uint64_t>(replay_launches_);
        complete_evaluation();
        after_evaluation(t0);
    } else {
        enqueue_positions(src, device_positions);
        evaluate();
    }
    account_evaluation(start);
}

void Evaluator::compute_xyz(std::uint64_t generation, const double* xyz, const double* r, bool device_arrays)
{
    const CallStart start;
    check_generation(generation);
    const long long E = num_edges_;
    if (tile_receivers_ > 0) {
        // the tiled plan copies each tile's slice of the caller's arrays into
        // its arena during this call; nothing is kept graph-wide
        explicit_xyz_ = xyz;
        explicit_r_ = r;
        explicit_device_ = device_arrays;
    } else {
        const hipMemcpyKind kind = device_arrays ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
        xyz_.reserve(static_cast<std::size_t>(std::max<long long>(E, 1)) * 3 * sizeof(double));
        r_.reserve(static_cast<std::size_t>(std::max<long long>(E, 1)) * sizeof(double));
        if (E > 0) {
            hip_check(hipMemcpyAsync(xyz_.as<double>(), xyz, E * 3 * sizeof(double), kind, stream_), "xyz");
            hip_check(hipMemcpyAsync(r_.as<double>(), r, E * sizeof(double), kind, stream_), "r");
        }
    }
    for (int i = 0; i < kNumStages; ++i) stage_used_[i] = false;
    check_geometry_ = false;
    explicit_geometry_ = true;
    try {
        evaluate();
    } catch (...) {
        explicit_xyz_ = explicit_r_ = nullptr;
        throw;
    }
    explicit_xyz_ = explicit_r_ = nullptr;
    account_evaluation(start);
}

double Evaluator::max_displacement(std::uint64_t generation, const double* positions, bool device_positions)
{
    return std::sqrt(max_displacement_squared(generation, positions, device_positions));
}

double Evaluator::max_displacement_squared(std::uint64_t generation, const double* positions, bool device_positions)
{
    require_geometry(generation);
    const int N = num_nodes_;
    if (N > 0 && positions != positions_.as<double>())
        hip_check(hipMemcpyAsync(positions_.as<double>(), positions, N * 3 * sizeof(double),
                                 device_positions ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, stream_),
                  "positions");
    const double* cell = cell_dev_.as<double>();
    hip_check(launch_atom_displacements(N, positions_.as<double>(), geometry_ref(), cell, cell + 9,
                                        disp_.as<double>(), totals_.as<double>() + 12, stream_),
              "displacement");
    double d2 = 0.0;
    hip_check(hipMemcpyAsync(&d2, totals_.as<double>() + 12, sizeof(double), hipMemcpyDeviceToHost, stream_),
              "copy");
    wait("displacement");
    return d2;
}

// Density-normalisation arguments of the layer and readout kernels.
void Evaluator::density_args(LayerArgs& la, ReadoutArgs* ra)
{
    la.d0 = DensityScale{};
    la.d1 = DensityScale{};
    if (model_.A0_scaled) la.d0.table = dens0_.as<float>();
    if (model_.A1_scaled) {
        la.d1.table = dens1_.as<float>();
        la.d1.scale = scale1_.as<float>();
        la.d1.dot = dot1_.as<float>();
    }
    if (ra) {
        ra->a1_scale = la.d1.scale;
        ra->a1_dot = la.d1.dot;
    }
}

// ZBL pair term over every receiver (after the forces of the MACE part).
void Evaluator::launch_zbl_term(const LayerArgs& la, double* forces, hipStream_t s)
{
    if (!model_.has_zbl) return;
    ZblArgs z;
    z.inverse_a = zbl_inverse_a_.as<double>();
    z.prefactor = zbl_prefactor_.as<double>();
    z.r_max = zbl_rmax_.as<double>();
    for (int q = 0; q < 4; ++q) z.c[q] = model_.zbl_c[q];
    z.p = model_.zbl_p;
    const EdgeGraph& g = la.graph;
    hip_check(launch_zbl(la.node_offset, la.node_count, g.first, g.edge_base, g.edge_pair, g.xyz, g.r, z,
                         energies_.as<double>(), forces, s),
              "ZBL");
}

// H1 = M0 H1_W per l block (+ the fused first-interaction residual of the
// node's element, mace_kokkos_h1_phi1.cpp:511-537) or, reverse, M0_adj =
// H1_adj H1_W^T, for `nodes` consecutive nodes from graph node `node_base`,
// one grouped launch.  With x_out (pre_linear_up basis, forward) the same
// launch forms the readout input x = M0_scalar P0 + residual_scalar
// (mace_kokkos_h1_phi1.cpp:253-280, 538-552).
void Evaluator::gemm_h1(int nodes, int node_base, const float* in, long long in_stride, float* out,
                        long long out_stride, bool reverse, float* x_out, const char* what)
{
    const long long type_stride = static_cast<long long>(nLM_) * C_;
    GemmGroup grp;
    for (int l = 0; l <= model_.L_max; ++l) {
        GemmArgs& g = grp.g[grp.count++];
        g.nodes = nodes;
        g.rows_per_node = 2 * l + 1;
        g.K = C_;
        g.Ncols = C_;
        g.a = {in + l * l * C_, in_stride, C_};
        // Bt = W^T for H1 = M0 W, and W for M0_adj = H1_adj W^T
        g.Bt = (reverse ? h1w_ : h1wt_).as<float>() + static_cast<std::size_t>(l) * C_ * C_;
        g.c = {out + l * l * C_, out_stride, C_};
        if (!reverse && model_.first_residual)
            g.bias = {residual_fused_.as<float>() + l * l * C_, node_types_.as<int>(), node_base, type_stride, C_};
    }
    if (x_out) {
        GemmArgs& g = grp.g[grp.count++];
        g.nodes = nodes;
        g.rows_per_node = 1;
        g.K = C_;
        g.Ncols = C_;
        g.a = {in, in_stride, C_};
        g.Bt = p0wt_.as<float>();
        g.c = {x_out, C_, C_};
        if (model_.first_residual)
            g.bias = {residual_.as<float>(), node_types_.as<int>(), node_base, type_stride, C_};
    }
    hip_check(launch_gemm_group(grp, stream_), what);
}

// M0_adj scalar block += the readout's direct adjoint of x: direct itself
// (m0_composite, x = M0_scalar) or direct P0^T (pre_linear_up, reference
// add_h1_affine_direct_adjoint, mace_kokkos_h1_phi1.cpp:296-345).
void Evaluator::add_direct(int nodes, int node_base, float* M0adj, hipStream_t s)
{
    const float* direct = (tile_receivers_ > 0 ? M0s_ : direct_).as<float>() + static_cast<std::size_t>(node_base) * C_;
    if (!model_.pre_linear_up) {
        hip_check(launch_add_direct(nodes, C_, nLM_, direct, M0adj, s), "direct adjoint");
        return;
    }
    GemmGroup grp;
    GemmArgs& g = grp.g[grp.count++];
    g.nodes = nodes;
    g.rows_per_node = 1;
    g.K = C_;
    g.Ncols = C_;
    g.a = {direct, C_, C_};
    g.Bt = p0w_.as<float>();  // M0_adj[kp] += sum_k P0[kp][k] direct[k]
    g.c = {M0adj, static_cast<long long>(nLM_) * C_, C_};
    g.accumulate = 1;
    hip_check(launch_gemm_group(grp, s), "direct adjoint");
}

// A0 = A0_pre A0_W[type, l] (reverse: A0_pre_adj = A0_adj A0_W[type, l]^T)
// per active type and l block over the untiled plan's nodes of that type
// (node_order_ groups them), up to kMaxGemmGroup GEMMs per launch.
void Evaluator::gemm_a0(const float* in, float* out, bool reverse)
{
    const int NL = model_.l_max + 1;
    const long long node_stride = static_cast<long long>(nlm_) * C_;
    const float* W = (reverse ? a0w_ : a0wt_).as<float>();
    GemmGroup grp;
    auto flush = [&] {
        if (grp.count > 0) hip_check(launch_gemm_group(grp, stream_), reverse ? "A0 reverse gemm" : "A0 gemm");
        grp = GemmGroup{};
    };
    for (std::size_t a = 0; a < active_types_.size(); ++a) {
        if (type_count_[a] == 0) continue;
        for (int l = 0; l < NL; ++l) {
            if (grp.count == kMaxGemmGroup) flush();
            GemmArgs& g = grp.g[grp.count++];
            g.nodes = type_count_[a];
            g.rows_per_node = 2 * l + 1;
            g.K = C_;
            g.Ncols = C_;
            g.a = {in + static_cast<std::size_t>(l) * l * C_, node_stride, C_};
            g.node_ids = node_order_.as<int>() + type_start_[a];
            g.Bt = W + (a * NL + l) * static_cast<std::size_t>(C_) * C_;
            g.c = {out + static_cast<std::size_t>(l) * l * C_, node_stride, C_};
        }
    }
    flush();
}

// A1[l] = Phi1[l group] A1_W[l] (or, reverse, dPhi1[l group] = A1_adj[l]
// A1_W[l]^T) for `nodes` consecutive tile-local nodes, one grouped launch.
void Evaluator::gemm_a1(int nodes, const float* in, float* out, bool reverse, const char* what)
{
    const long long nodelm = static_cast<long long>(nlm_) * C_;
    const long long nodelme = static_cast<long long>(nlme_) * C_;
    GemmGroup grp;
    for (int l = 0; l <= model_.l_max; ++l) {
        if (num_e_[l] == 0) continue;
        GemmArgs& g = grp.g[grp.count++];
        const long long phi_row = static_cast<long long>(num_e_[l]) * C_;
        g.nodes = nodes;
        g.rows_per_node = 2 * l + 1;
        if (!reverse) {
            g.K = num_e_[l] * C_;
            g.Ncols = C_;
            g.a = {in + static_cast<long long>(lme_off_[l]) * C_, nodelme, phi_row};
            g.Bt = a1wt_[l]->as<float>();
            g.c = {out + l * l * C_, nodelm, C_};
        } else {
            g.K = C_;
            g.Ncols = num_e_[l] * C_;
            g.a = {in + l * l * C_, nodelm, C_};
            g.Bt = a1w_[l]->as<float>();
            g.c = {out + static_cast<long long>(lme_off_[l]) * C_, nodelme, phi_row};
        }
    }
    hip_check(launch_gemm_group(grp, stream_), what);
}

void Evaluator::evaluate()
{
    if (tile_receivers_ > 0) {
        evaluate_tiled();
        return;
    }
    const auto t0 = std::chrono::steady_clock::now();
    enqueue_evaluation();
    // the evaluation (and any copy from caller-owned host arrays) has completed
    // when this returns
    finish_evaluation();
    after_evaluation(t0);
}

// Per-stage times, the evaluated generation and the call's statistics once
// an untiled evaluation has completed.
void Evaluator::after_evaluation(std::chrono::steady_clock::time_point t0)
{
    if (profiling_)
        for (int i = 0; i < kNumStages; ++i) {
            if (!stage_used_[i]) continue;
            float ms = 0.0f;
            hip_check(hipEventElapsedTime(&ms, events_[2 * i], events_[2 * i + 1]), "event time");
            stage_ms_[i] += ms;
            stage_count_[i] += 1;
        }
    evaluated_generation_ = generation_;
    reduced_ = fused_volume_ > 0.0;
    reduced_volume_ = fused_volume_;
    stats_.evaluations += 1;
    stats_.last_evaluation_ms =
        std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

// The untiled evaluation's kernels, from the layer-0 edge pass to the atom
// forces, on the evaluator's stream (no host wait).
void Evaluator::enqueue_evaluation()
{
    const int N = num_nodes_;
    const int E = static_cast<int>(num_edges_);
    LayerArgs la;
    la.graph.num_nodes = N;
    la.graph.num_edges = E;
    la.graph.node_types = node_types_.as<int>();
    la.graph.type_active = type_active_.as<int>();
    la.graph.num_active = static_cast<int>(active_types_.size());
    la.graph.first = first_.as<int>();
    la.graph.receiver = receiver_.as<int>();
    la.graph.source = source_.as<int>();
    la.graph.tfirst = tfirst_.as<int>();
    la.graph.tedge = tedge_.as<int>();
    la.graph.edge_pair = edge_pair_.as<int>();
    la.graph.xyz = xyz_.as<double>();
    la.graph.r = r_.as<double>();
    la.grid = grid_;
    la.C = C_;
    la.l_max = model_.l_max;
    la.L_max = model_.L_max;
    la.channel_slices = r1_graph_slices_;
    la.reverse_slices = r1_rev_slices_;
    la.a0_slices = a0_graph_slices_;
    la.node_offset = 0;
    la.node_count = N;
    if (num_edge_tiles_ > 0) {
        la.edge_tiles = edge_tiles_.as<int>();
        la.edge_tiles_layer0 = edge_tiles_l0_.as<int>();
        la.num_edge_tiles = num_edge_tiles_;
        la.edge_tile = edge_tile_;
    }
    density_args(la, nullptr);
    la.type_order = node_order_.as<int>();
    hipStream_t s = stream_;
    const PolyArgs p0 = poly_args(p0_layout_, p0_coef_, p0_offsets_, p0_packed_);
    const PolyArgs p1 = poly_args(p1_layout_, p1_coef_, p1_offsets_, p1_packed_);
    const long long nodeLM = static_cast<long long>(nLM_) * C_;

    if (E > 0 || N > 0) {
        // layer 0: A0 (folded H0, A0_W), M0, H1
        mark(kStageA0Forward, false);
        if (a0_unfolded()) {
            LayerArgs lu = la;
            lu.h0 = h0s_.as<float>();
            hip_check(launch_a0_forward(lu, r0u_.as<float>(), A0pre_.as<float>(), s), "A0 forward");
            gemm_a0(A0pre_.as<float>(), A0_.as<float>(), false);
        } else {
            hip_check(launch_a0_forward(la, r0f_.as<float>(), A0_.as<float>(), s), "A0 forward");
        }
        mark(kStageA0Forward, true);
        mark(kStageM0Forward, false);
        hip_check(launch_m0_forward(la, p0, node_blocks(m0_blocks_, m0_block_offsets_, 0, m0_block_nodes_), A0_.as<float>(),
                                    M0_.as<float>(), s),
                  "M0 forward");
        mark(kStageM0Forward, true);
        mark(kStageH1Gemm, false);
        gemm_h1(N, 0, M0_.as<float>(), nodeLM, H1_.as<float>(), nodeLM, false,
                model_.pre_linear_up ? M0s_.as<float>() : nullptr, "H1 gemm");
        mark(kStageH1Gemm, true);
        // layer 1: Phi1 -> A1
        mark(kStageR1Forward, false);
        hip_check(launch_r1_forward(la, r1_.as<float>(), cg_.as<float>(), H1_.as<float>(), Phi1_.as<float>(), s),
                  "R1 forward");
        mark(kStageR1Forward, true);
        mark(kStageA1Gemm, false);
        gemm_a1(N, Phi1_.as<float>(), A1_.as<float>(), false, "A1 gemm");
        mark(kStageA1Gemm, true);
        // readout and its reverse down to A1_adj
        ReadoutArgs ra;
        ra.nodes = node_blocks(readout_blocks_, readout_block_offsets_, 0, readout_block_nodes_);
        ra.local_base = 0;
        ra.m0_stride = nodeLM;
        ra.C = C_;
        ra.num_lm = nlm_;
        ra.num_LM = nLM_;
        ra.hidden = model_.readout_hidden;
        ra.node_types = node_types_.as<int>();
        ra.type_active = type_active_.as<int>();
        ra.A1 = A1_.as<float>();
        if (model_.pre_linear_up) {
            ra.M0 = M0s_.as<float>();
            ra.m0_stride = C_;
        } else {
            ra.M0 = M0_.as<float>();
        }
        ra.p1 = p1;
        ra.H2M0 = h2m0_.as<float>();
        ra.H2M0T = h2m0t_.as<float>();
        ra.H2M1 = h2m1_.as<float>();
        ra.H2M1T = h2m1t_.as<float>();
        ra.q = q_.as<float>();
        ra.W1 = w1_.as<float>();
        ra.W2 = w2_.as<float>();
        ra.scale = static_cast<float>(model_.readout_scale);
        ra.E0 = e0_.as<double>();
        ra.energies = energies_.as<double>();
        ra.direct = direct_.as<float>();
        ra.A1_adj = A1adj_.as<float>();
        density_args(la, &ra);
        mark(kStageReadout, false);
        hip_check(launch_readout(ra, s), "readout");
        mark(kStageReadout, true);
        mark(kStageA1ReverseGemm, false);
        // dPhi1 = A1_adj A1_W^T  (into the Phi1 buffer, no longer needed)
        float* dPhi1 = Phi1_.as<float>();
        gemm_a1(N, A1adj_.as<float>(), dPhi1, true, "A1 reverse gemm");
        mark(kStageA1ReverseGemm, true);
        mark(kStageR1Reverse, false);
        hip_check(launch_r1_reverse(la, r1_.as<float>(), cg_.as<float>(), H1_.as<float>(), dPhi1,
                                    forces_.as<double>(), msg_.as<float>(), rpart_.as<double>(), s),
                  "R1 reverse");
        mark(kStageR1Reverse, true);
        mark(kStageGather, false);
        hip_check(launch_gather_messages(la, msg_.as<float>(), H1adj_.as<float>(), s), "H1 adjoint gather");
        mark(kStageGather, true);
        mark(kStageH1ReverseGemm, false);
        // M0_adj = H1_adj H1_W^T (+ direct scalar adjoint), into the M0 buffer
        float* M0adj = M0_.as<float>();
        gemm_h1(N, 0, H1adj_.as<float>(), nodeLM, M0adj, nodeLM, true, nullptr, "H1 reverse gemm");
        add_direct(N, 0, M0adj, s);
        mark(kStageH1ReverseGemm, true);
        // A0_adj into the A1 buffer (no longer needed)
        float* A0adj = A1_.as<float>();
        mark(kStageM0Reverse, false);
        hip_check(launch_m0_reverse(la, p0, node_blocks(m0r_blocks_, m0r_block_offsets_, 0, m0r_block_nodes_), A0_.as<float>(), M0adj,
                                    A0adj, s),
                  "M0 reverse");
        mark(kStageM0Reverse, true);
        mark(kStageA0Reverse, false);
        if (a0_unfolded()) {
            // the adjoint of the sums before A0_W, into the Phi1 buffer (dPhi1
            // is consumed); A0_adj . A0 = A0pre_adj . A0pre for the density term
            float* A0pre_adj = Phi1_.as<float>();
            gemm_a0(A0adj, A0pre_adj, true);
            LayerArgs lu = la;
            lu.h0 = h0s_.as<float>();
            hip_check(launch_a0_reverse(lu, r0u_.as<float>(), A0pre_.as<float>(), A0pre_adj, forces_.as<double>(), s),
                      "A0 reverse");
        } else {
            hip_check(launch_a0_reverse(la, r0f_.as<float>(), A0_.as<float>(), A0adj, forces_.as<double>(), s),
                      "A0 reverse");
        }
        mark(kStageA0Reverse, true);
        launch_zbl_term(la, forces_.as<double>(), s);
    }
    mark(kStageAtomForces, false);
    hip_check(launch_atom_forces(N, first_.as<int>(), tfirst_.as<int>(), tedge_.as<int>(), forces_.as<double>(),
                                 atom_forces_.as<double>(), s),
              "atom forces");
    mark(kStageAtomForces, true);
}

// Tiled evaluation (reference compute_dual_layer_tiled,
// mace_kokkos_evaluate.cpp:754-1238): three sweeps over receiver tiles with
// one reused arena.  The arena holds the tile's receiver work arrays and, per
// tile edge, its geometry, pair code, directed force and H1-adjoint message;
// graph-wide state is per node (H1, its adjoint, the scalar M0 block, the
// direct adjoint, energies, atom forces) plus the sources, cell shifts and
// source-major edge list.
//   1. edge geometry -> A0 -> M0 -> H1 (graph-wide), keeping the scalar M0
//      block graph-wide;
//   2. edge geometry -> Phi1 -> A1 -> readout (energies, direct adjoint) ->
//      dPhi1 -> R1 reverse (directed forces, messages) -> H1 adjoint += the
//      tile's messages, run by run; the directed forces are folded into the
//      atom forces and the virial;
//   3. edge geometry -> M0 adjoint = H1 adjoint H1_W^T + direct -> A0
//      (recomputed) -> A0 adjoint -> A0 reverse (+ ZBL) directed forces,
//      folded likewise.
// Each tile's edges are its receivers' contiguous CSR range.  Atom forces and
// the virial are linear in the directed forces, so folding the two sweeps'
// parts separately gives the same totals; the fold order is fixed (receiver
// part, then the tile's source runs), so results are run-to-run identical.
void Evaluator::evaluate_tiled()
{
    const auto t0 = std::chrono::steady_clock::now();
    const int N = num_nodes_;
    const int T = tile_receivers_;
    LayerArgs la;
    la.graph.num_nodes = N;
    la.graph.node_types = node_types_.as<int>();
    la.graph.type_active = type_active_.as<int>();
    la.graph.num_active = static_cast<int>(active_types_.size());
    la.graph.receiver = nullptr;  // not kept by the tiled plan
    la.graph.tfirst = nullptr;
    la.graph.edge_pair = tile_pair_.as<int>();
    la.graph.xyz = tile_xyz_.as<double>();
    la.graph.r = tile_r_.as<double>();
    la.graph.edge_base = 0;  // every edge array is passed from the tile's first edge on
    la.grid = grid_;
    la.C = C_;
    la.l_max = model_.l_max;
    la.L_max = model_.L_max;
    la.channel_slices = r1_slices_;
    la.reverse_slices = r1_rev_slices_;
    density_args(la, nullptr);
    la.type_order = node_order_.as<int>();
    hipStream_t s = stream_;
    const PolyArgs p0 = poly_args(p0_layout_, p0_coef_, p0_offsets_, p0_packed_);
    const PolyArgs p1 = poly_args(p1_layout_, p1_coef_, p1_offsets_, p1_packed_);
    const long long nodeLM = static_cast<long long>(nLM_) * C_;
    double* forces = tile_forces_.as<double>();
    double* atom_forces = atom_forces_.as<double>();
    double* virial = totals_.as<double>() + 16;  // [16] unused, [17..25] -sum f (x) xyz
    // the tile's geometry: the caller's edge vectors, or the prepared
    // geometry with the displacements of this evaluation
    const bool in_arena = explicit_geometry_;
    if (in_arena && num_edges_ > 0 && !(explicit_xyz_ && explicit_r_))
        throw std::logic_error("tiled evaluation from edge vectors without the caller's arrays");
    const GeometryRef ref = in_arena ? GeometryRef{} : geometry_ref();
    TileGeometry tg;
    tg.node_types = node_types_.as<int>();
    tg.type_active = type_active_.as<int>();
    tg.num_active = static_cast<int>(active_types_.size());
    tg.shared_tables = shared_pair_tables();
    tg.in_arena = in_arena;
    tg.disp = disp_.as<double>();
    tg.cell = cell_dev_.as<double>();
    tg.r_cut = model_.r_cut;
    tg.xyz = tile_xyz_.as<double>();
    tg.r = tile_r_.as<double>();
    tg.edge_pair = tile_pair_.as<int>();
    tg.edge_base = 0;
    auto tile = [&](int t, bool count_invalid) {
        // tile-local offsets (first_ + t, indexed by graph receiver ids) and
        // the graph-wide edge arrays from the tile's first edge on
        const long long base = tile_first_edge_[t];
        const long long tile_edges = tile_first_edge_[t + 1] - base;
        la.node_offset = t * T;
        la.node_count = std::min(T, N - t * T);
        la.local_base = la.node_offset;
        la.graph.num_edges = static_cast<int>(tile_edges);
        la.graph.first = first_.as<int>() + t;
        la.graph.source = source_.as<int>() + base;
        la.graph.tedge = tedge_.as<int>() + base;
        tg.node_begin = la.node_offset;
        tg.node_count = la.node_count;
        tg.first = la.graph.first;
        tg.source = la.graph.source;
        tg.pair_source = pair_from_types_ ? nullptr : edge_pair_.as<int>() + base;
        tg.ref = ref;
        if (ref.edges) tg.ref.edges = ref.edges + 3 * base;
        if (ref.shifts) tg.ref.shifts = ref.shifts + 3 * base;
        if (ref.shifts8) tg.ref.shifts8 = ref.shifts8 + 3 * base;
        tg.invalid = count_invalid && check_geometry_
                         ? reinterpret_cast<unsigned long long*>(totals_.as<double>() + 13)
                         : nullptr;
        if (in_arena && tile_edges > 0) {
            const hipMemcpyKind kind = explicit_device_ ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
            hip_check(hipMemcpyAsync(tile_xyz_.as<double>(), explicit_xyz_ + 3 * base,
                                     static_cast<std::size_t>(tile_edges) * 3 * sizeof(double), kind, s),
                      "tile xyz");
            hip_check(hipMemcpyAsync(tile_r_.as<double>(), explicit_r_ + base,
                                     static_cast<std::size_t>(tile_edges) * sizeof(double), kind, s),
                      "tile r");
        }
        hip_check(launch_tile_geometry(tg, s), "tile geometry");
    };
    auto runs_of = [&](int t) {
        TileRuns runs;
        runs.count = tile_run_offsets_[t + 1] - tile_run_offsets_[t];
        runs.source = run_source_.as<int>() + tile_run_offsets_[t];
        runs.start = run_start_.as<int>() + tile_run_offsets_[t];
        runs.length = run_length_.as<int>() + tile_run_offsets_[t];
        return runs;
    };
    // the tile's directed forces into the atom forces and the virial
    auto fold = [&](int t) {
        const long long tile_edges = tile_first_edge_[t + 1] - tile_first_edge_[t];
        hip_check(launch_fold_tile_forces(la.node_offset, la.node_count, la.graph.first, runs_of(t), la.graph.tedge,
                                          0, forces, atom_forces, s),
                  "fold forces");
        if (tile_edges > 0) {
            const int np = reduce_totals_partials(0, static_cast<int>(tile_edges));
            hip_check(launch_reduce_totals(0, static_cast<int>(tile_edges), nullptr, forces, tile_xyz_.as<double>(),
                                           1.0, partials_.as<double>(), np, virial, s, true),
                      "virial");
        }
    };
    float* H1 = H1_.as<float>();
    float* H1adj = H1adj_.as<float>();
    float* M0s = M0s_.as<float>();
    hip_check(hipMemsetAsync(H1adj, 0, static_cast<std::size_t>(N) * nodeLM * sizeof(float), s), "memset");
    hip_check(launch_fill_f64(atom_forces, 3LL * N, 0.0, s), "clear forces");
    hip_check(launch_fill_f64(virial, 10, 0.0, s), "clear virial");
    // sweep 1
    for (int t = 0; t < num_tiles_; ++t) {
        tile(t, true);
        hip_check(launch_a0_forward(la, r0f_.as<float>(), A0_.as<float>(), s), "A0 forward");
        hip_check(launch_m0_forward(la, p0, node_blocks(m0_blocks_, m0_block_offsets_, t, m0_block_nodes_), A0_.as<float>(),
                                    M0_.as<float>(), s),
                  "M0 forward");
        float* x = M0s + static_cast<std::size_t>(la.node_offset) * C_;
        gemm_h1(la.node_count, la.node_offset, M0_.as<float>(), nodeLM, H1 + la.node_offset * nodeLM, nodeLM, false,
                model_.pre_linear_up ? x : nullptr, "H1 gemm");
        if (!model_.pre_linear_up)
            hip_check(hipMemcpy2DAsync(x, C_ * sizeof(float), M0_.as<float>(), nodeLM * sizeof(float),
                                       C_ * sizeof(float), la.node_count, hipMemcpyDeviceToDevice, s),
                      "M0 scalar block");
    }
    // sweep 2
    ReadoutArgs ra;
    ra.C = C_;
    ra.num_lm = nlm_;
    ra.num_LM = nLM_;
    ra.hidden = model_.readout_hidden;
    ra.node_types = node_types_.as<int>();
    ra.type_active = type_active_.as<int>();
    ra.A1 = A1_.as<float>();
    ra.M0 = M0s;
    ra.m0_stride = C_;
    ra.p1 = p1;
    ra.H2M0 = h2m0_.as<float>();
    ra.H2M0T = h2m0t_.as<float>();
    ra.H2M1 = h2m1_.as<float>();
    ra.H2M1T = h2m1t_.as<float>();
    ra.q = q_.as<float>();
    ra.W1 = w1_.as<float>();
    ra.W2 = w2_.as<float>();
    ra.scale = static_cast<float>(model_.readout_scale);
    ra.E0 = e0_.as<double>();
    ra.energies = energies_.as<double>();
    ra.direct = M0s;  // over each node's scalar block, once the readout has read it
    ra.A1_adj = A1adj_.as<float>();
    density_args(la, &ra);
    float* dPhi1 = Phi1_.as<float>();
    for (int t = 0; t < num_tiles_; ++t) {
        tile(t, false);
        hip_check(launch_r1_forward(la, r1_.as<float>(), cg_.as<float>(), H1, Phi1_.as<float>(), s), "R1 forward");
        gemm_a1(la.node_count, Phi1_.as<float>(), A1_.as<float>(), false, "A1 gemm");
        ra.nodes = node_blocks(readout_blocks_, readout_block_offsets_, t, readout_block_nodes_);
        ra.local_base = la.local_base;
        hip_check(launch_readout(ra, s), "readout");
        gemm_a1(la.node_count, A1adj_.as<float>(), dPhi1, true, "A1 reverse gemm");
        hip_check(launch_r1_reverse(la, r1_.as<float>(), cg_.as<float>(), H1, dPhi1, forces, msg_.as<float>(),
                                    rpart_.as<double>(), s),
                  "R1 reverse");
        hip_check(launch_gather_tile_runs(la, runs_of(t), msg_.as<float>(), H1adj, s), "H1 adjoint gather");
        fold(t);
    }
    // sweep 3
    float* M0adj = M0_.as<float>();
    float* A0adj = A1_.as<float>();
    for (int t = 0; t < num_tiles_; ++t) {
        tile(t, false);
        gemm_h1(la.node_count, la.node_offset, H1adj + la.node_offset * nodeLM, nodeLM, M0adj, nodeLM, true, nullptr,
                "H1 reverse gemm");
        add_direct(la.node_count, la.node_offset, M0adj, s);
        hip_check(launch_a0_forward(la, r0f_.as<float>(), A0_.as<float>(), s), "A0 forward");
        hip_check(launch_m0_reverse(la, p0, node_blocks(m0r_blocks_, m0r_block_offsets_, t, m0r_block_nodes_), A0_.as<float>(), M0adj,
                                    A0adj, s),
                  "M0 reverse");
        // the A0 reverse adds into the directed forces: this sweep's part starts at zero
        const long long tile_edges = tile_first_edge_[t + 1] - tile_first_edge_[t];
        hip_check(launch_fill_f64(forces, 3 * tile_edges, 0.0, s), "clear tile forces");
        hip_check(launch_a0_reverse(la, r0f_.as<float>(), A0_.as<float>(), A0adj, forces, s), "A0 reverse");
        launch_zbl_term(la, forces, s);
        fold(t);
    }
    finish_evaluation();
    evaluated_generation_ = generation_;
    reduced_ = fused_volume_ > 0.0;
    reduced_volume_ = fused_volume_;
    stats_.evaluations += 1;
    stats_.tiled_evaluations += 1;
    stats_.last_evaluation_ms =
        std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

// 1 eV / (A amu) in A / fs^2
constexpr double kForceToAcceleration = 9.648533212e-3;

// Velocity-Verlet NVE (the LAMMPS `fix nve` update the reference's capacity
// runs use with pair_style symmetrix/mace): per step v += dt/2 a, x += dt v,
// forces at the new positions, v += dt/2 a.  Every array stays on the
// device.  The second half kick and the kinetic energy are queued behind
// the evaluation at the new positions, and the squared displacement that
// evaluation measured decides whether the graph still held, on the device
// (the kick applies only if it did) and on the host afterwards with the same
// comparison; if not, the graph is rebuilt and the evaluation and kick run
// again on the unkicked velocities.  While the displacement since the build
// plus twice its largest growth per step so far stays below skin/2, a step
// evaluates on the graph directly and waits on the host once; otherwise
// (the first step, the steps near a rebuild) the displacement is checked
// before the evaluation, so an evaluation is rarely run on a graph that no
// longer holds (which would cost a whole evaluation at capacity sizes).
int Evaluator::md_nve(int num_atoms, const int* node_types, const double* masses, double* x, double* v,
                      const double* cell, const double* inverse_cell, double skin, double dt, int steps,
                      double* epot, double* ekin, double* step_seconds)
{
    if (num_atoms <= 0) throw std::invalid_argument("MD requires at least one atom");
    if (steps < 0) throw std::invalid_argument("MD step count must be non-negative");
    if (!std::isfinite(dt) || !(dt > 0.0)) throw std::invalid_argument("MD time step must be finite and positive");
    if (!std::isfinite(skin) || skin < 0.0) throw std::invalid_argument("neighbor skin must be finite and non-negative");
    const int N = num_atoms;
    std::vector<double> m(masses, masses + N), inv_m(N);
    for (int a = 0; a < N; ++a) {
        if (!std::isfinite(m[a]) || !(m[a] > 0.0)) throw std::invalid_argument("MD masses must be finite and positive");
        inv_m[a] = kForceToAcceleration / m[a];
    }
    const std::size_t bytes3 = static_cast<std::size_t>(N) * 3 * sizeof(double);
    md_x_.reserve(bytes3);
    md_v_.reserve(bytes3);
    hip_check(hipMemcpyAsync(md_x_.as<double>(), x, bytes3, hipMemcpyHostToDevice, stream_), "MD positions");
    hip_check(hipMemcpyAsync(md_v_.as<double>(), v, bytes3, hipMemcpyHostToDevice, stream_), "MD velocities");
    upload(md_m_, m, stream_, &staged_);
    upload(md_inv_m_, inv_m, stream_, &staged_);
    const int np = md_kinetic_partials(N);
    md_partials_.reserve(static_cast<std::size_t>(np) * sizeof(double));
    double* xd = md_x_.as<double>();
    double* vd = md_v_.as<double>();
    const double cutoff = model_.r_cut + skin;
    // the graph holds while every atom moved at most skin/2 since its build:
    // squared displacement (totals_[12]) <= (skin/2)^2
    const double limit2 = (0.5 * skin) * (0.5 * skin);
    // the kinetic energy of `vel`, queued on the stream: m |v|^2 lands in
    // totals_[14] and host_totals_[14]
    auto queue_kinetic = [&](const double* vel) {
        hip_check(launch_md_kinetic(N, vel, md_m_.as<double>(), md_partials_.as<double>(), np,
                                    totals_.as<double>() + 14, stream_),
                  "kinetic energy");
        hip_check(hipMemcpyAsync(host_totals_ + 14, totals_.as<double>() + 14, sizeof(double), hipMemcpyDeviceToHost,
                                 stream_),
                  "copy");
    };
    struct EpilogueGuard {
        std::function<void()>& slot;
        ~EpilogueGuard() { slot = nullptr; }
    } guard{epilogue_};

    std::uint64_t gen = prepare_periodic_graph(N, node_types, xd, true, cell, inverse_cell, cutoff);
    int rebuilds = 0;
    epilogue_ = [&] { queue_kinetic(vd); };
    compute_positions(gen, xd, true);
    epilogue_ = nullptr;
    if (epot) epot[0] = total_energy(gen);
    if (ekin) ekin[0] = 0.5 * host_totals_[14] / kForceToAcceleration;
    const double dtf = 0.5 * dt;
    double disp = 0.0;      // displacement since the graph's build after the last evaluation
    double growth = -1.0;   // largest growth of it in one step (negative: none seen yet)
    for (int step = 1; step <= steps; ++step) {
        const auto t0 = std::chrono::steady_clock::now();
        hip_check(launch_md_kick_drift(N, xd, vd, atom_forces_.as<double>(), md_inv_m_.as<double>(), dtf, dt, stream_),
                  "MD drift");
        bool rebuilt = false;
        if (!(growth >= 0.0 && disp + 2.0 * growth < 0.5 * skin)) {
            // near a rebuild (or no growth seen yet): check before evaluating
            if (!(max_displacement_squared(gen, xd, true) <= limit2)) {
                gen = prepare_periodic_graph(N, node_types, xd, true, cell, inverse_cell, cutoff);
                ++rebuilds;
                rebuilt = true;
            }
        }
        epilogue_ = [&] {
            hip_check(launch_md_kick(N, vd, atom_forces_.as<double>(), md_inv_m_.as<double>(), dtf,
                                     totals_.as<double>() + 12, limit2, stream_),
                      "MD kick");
            if (ekin) queue_kinetic(vd);
        };
        compute_positions(gen, xd, true);
        if (!(host_totals_[12] <= limit2)) {
            // the graph no longer covers every pair within the cutoff (the
            // kick did not apply): rebuild and evaluate again
            gen = prepare_periodic_graph(N, node_types, xd, true, cell, inverse_cell, cutoff);
            ++rebuilds;
            rebuilt = true;
            compute_positions(gen, xd, true);
        }
        epilogue_ = nullptr;
        const double now = std::sqrt(host_totals_[12]);
        if (!rebuilt) growth = std::max(growth, now - disp);
        disp = now;
        double seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        if (step_seconds) step_seconds[step - 1] = seconds;
        if (epot) epot[step] = total_energy(gen);
        if (ekin) ekin[step] = 0.5 * host_totals_[14] / kForceToAcceleration;
        if (md_progress_) {
            const double nan = std::numeric_limits<double>::quiet_NaN();
            if (md_progress_(step, epot ? epot[step] : nan, ekin ? ekin[step] : nan, seconds, md_progress_user_) != 0)
                break;
        }
    }
    hip_check(hipMemcpyAsync(x, xd, bytes3, hipMemcpyDeviceToHost, stream_), "MD positions");
    hip_check(hipMemcpyAsync(v, vd, bytes3, hipMemcpyDeviceToHost, stream_), "MD velocities");
    wait("MD");
    return rebuilds;
}

// Waits for the evaluation; an evaluation from positions raises when the
// edge geometry held an edge of zero or non-finite length (reference
// validate_prepared_factorized_positions_geometry,
// mace_kokkos_factorized_lifecycle.cpp:3078-3085).
// Volume of the current cell (0 for a non-finite determinant).
double Evaluator::cell_volume() const
{
    const double* c = cell_;
    const double v = std::abs(c[0] * (c[4] * c[8] - c[5] * c[7]) - c[1] * (c[3] * c[8] - c[5] * c[6]) +
                              c[2] * (c[3] * c[7] - c[4] * c[6]));
    return std::isfinite(v) ? v : 0.0;
}

// The totals kernels of an evaluation: the energy over the nodes and, for
// an untiled evaluation from positions in a cell of positive volume, the
// stress for that cell in the same pass (no host wait; part of a captured
// replay graph).
void Evaluator::enqueue_totals()
{
    const double volume = cell_volume();
    if (tile_receivers_ > 0) {
        // the energy over the nodes; the virial was accumulated tile by tile
        const int np = reduce_totals_partials(num_nodes_, 0);
        hip_check(launch_reduce_totals(num_nodes_, 0, energies_.as<double>(), nullptr, nullptr, 1.0,
                                       partials_.as<double>(), np, totals_.as<double>(), stream_),
                  "totals");
    } else if (check_geometry_ && volume > 0.0) {
        const int np = reduce_totals_partials(num_nodes_, static_cast<int>(num_edges_));
        hip_check(launch_reduce_totals(num_nodes_, static_cast<int>(num_edges_), energies_.as<double>(),
                                       forces_.as<double>(), xyz_.as<double>(), 1.0 / volume,
                                       partials_.as<double>(), np, totals_.as<double>(), stream_),
                  "totals");
    }
}

void Evaluator::finish_evaluation()
{
    enqueue_totals();
    complete_evaluation();
}

// Copies the totals (with the displacement maximum and the invalid-edge
// count) and, for host callers, the node energies and atom forces back, waits
// for the stream and checks the evaluation's edges.
void Evaluator::complete_evaluation()
{
    if (epilogue_) epilogue_();
    host_results_ = false;
    invalid_edges_ = 0;
    fused_volume_ = 0.0;
    last_from_positions_ = check_geometry_;
    const bool tiled = tile_receivers_ > 0;
    const double volume = cell_volume();
    const bool fuse = check_geometry_ && volume > 0.0;
    if (tiled) {
        hip_check(hipMemcpyAsync(host_totals_, totals_.as<double>(), 26 * sizeof(double), hipMemcpyDeviceToHost,
                                 stream_),
                  "totals copy");
    } else if (check_geometry_) {
        if (fuse) fused_volume_ = volume;
        hip_check(hipMemcpyAsync(host_totals_, totals_.as<double>(), 14 * sizeof(double), hipMemcpyDeviceToHost,
                                 stream_),
                  "totals copy");
    }
    const bool to_host = results_to_host_ && num_nodes_ > 0;
    if (to_host) {
        const std::size_t n = static_cast<std::size_t>(num_nodes_);
        pinned_energies_.reserve(n * sizeof(double));
        pinned_forces_.reserve(n * 3 * sizeof(double));
        hip_check(hipMemcpyAsync(pinned_energies_.as<double>(), energies_.as<double>(), n * sizeof(double),
                                 hipMemcpyDeviceToHost, stream_),
                  "energies copy");
        hip_check(hipMemcpyAsync(pinned_forces_.as<double>(), atom_forces_.as<double>(), n * 3 * sizeof(double),
                                 hipMemcpyDeviceToHost, stream_),
                  "forces copy");
    }
    results_to_host_ = false;
    wait("evaluation");
    if (tiled) {
        for (int q = 0; q < 9; ++q) host_virial_[q] = host_totals_[17 + q];
        if (fuse) {
            set_stress_from_virial(volume);
            fused_volume_ = volume;
        }
    }
    if (check_geometry_) std::memcpy(&invalid_edges_, host_totals_ + 13, sizeof(invalid_edges_));
    if (check_geometry_ && invalid_edges_ != 0) {
        check_geometry_ = false;
        evaluated_generation_ = 0;
        throw std::invalid_argument("Execution R1 prepared positions produced an invalid edge geometry.");
    }
    host_results_ = to_host;
}

// Tiled plan: stress = (-sum_e f_e (x) xyz_e) / V on the host, also written
// to the device totals (device results hold the last reduced stress).
void Evaluator::set_stress_from_virial(double volume)
{
    for (int q = 0; q < 9; ++q) host_totals_[1 + q] = host_virial_[q] / volume;
    // copied from a staged copy: no wait here, the stream orders it before
    // any later read of the device totals
    const auto* b = reinterpret_cast<const unsigned char*>(host_totals_ + 1);
    staged_.emplace_back(b, b + 9 * sizeof(double));
    hip_check(hipMemcpyAsync(totals_.as<double>() + 1, staged_.back().data(), 9 * sizeof(double),
                             hipMemcpyHostToDevice, stream_),
              "stress copy");
}

// Energy and stress totals of the completed evaluation for `volume`, in
// host_totals_ (reused when already reduced for this volume).
void Evaluator::reduce(double volume)
{
    if (evaluated_generation_ != generation_)
        throw std::invalid_argument("results require a completed evaluation of the current graph");
    if (reduced_ && reduced_volume_ == volume) return;
    if (!std::isfinite(volume) || !(volume > 0.0))
        throw std::invalid_argument("Stress reduction requires a positive finite volume.");
    if (tile_receivers_ > 0) {  // energy and virial are on the host already
        set_stress_from_virial(volume);
        reduced_ = true;
        reduced_volume_ = volume;
        return;
    }
    const int np = reduce_totals_partials(num_nodes_, static_cast<int>(num_edges_));
    hip_check(launch_reduce_totals(num_nodes_, static_cast<int>(num_edges_), energies_.as<double>(),
                                   forces_.as<double>(), xyz_.as<double>(), 1.0 / volume, partials_.as<double>(), np,
                                   totals_.as<double>(), stream_),
              "totals");
    hip_check(hipMemcpyAsync(host_totals_, totals_.as<double>(), 10 * sizeof(double), hipMemcpyDeviceToHost, stream_),
              "totals copy");
    synchronize();
    reduced_ = true;
    reduced_volume_ = volume;
}

double Evaluator::last_max_displacement() const
{
    if (!last_from_positions_ || evaluated_generation_ != generation_ || generation_ == 0)
        throw std::invalid_argument("no completed evaluation from positions of the current graph");
    return std::sqrt(host_totals_[12]);
}

void Evaluator::synchronize() const { hip_check(host_fence(stream_), "synchronize"); }

void Evaluator::node_energies(double* out) const
{
    if (evaluated_generation_ != generation_) throw std::invalid_argument("no completed evaluation");
    if (host_results_) {
        std::memcpy(out, pinned_energies_.as<double>(), static_cast<std::size_t>(num_nodes_) * sizeof(double));
        return;
    }
    if (num_nodes_ > 0)
        hip_check(hipMemcpyAsync(out, energies_.as<double>(), num_nodes_ * sizeof(double), hipMemcpyDeviceToHost,
                                 stream_),
                  "copy");
    synchronize();
}

void Evaluator::node_forces(double* out) const
{
    if (evaluated_generation_ != generation_) throw std::invalid_argument("no completed evaluation");
    if (tile_receivers_ > 0)
        throw std::invalid_argument(
            "The tiled plan folds directed edge forces into atom forces tile by tile and does not keep them; "
            "use the reduced atom forces.");
    if (num_edges_ > 0)
        hip_check(hipMemcpyAsync(out, forces_.as<double>(), num_edges_ * 3 * sizeof(double), hipMemcpyDeviceToHost,
                                 stream_),
                  "copy");
    synchronize();
}

void Evaluator::atom_forces(std::uint64_t generation, double* out)
{
    check_generation(generation);
    if (evaluated_generation_ != generation_)
        throw std::invalid_argument("Atom-force reduction requires the current completed graph.");
    if (host_results_) {
        std::memcpy(out, pinned_forces_.as<double>(), static_cast<std::size_t>(num_nodes_) * 3 * sizeof(double));
        return;
    }
    if (num_nodes_ > 0)
        hip_check(hipMemcpyAsync(out, atom_forces_.as<double>(), num_nodes_ * 3 * sizeof(double),
                                 hipMemcpyDeviceToHost, stream_),
                  "copy");
    synchronize();
}

void Evaluator::stress(std::uint64_t generation, double volume, double* out9)
{
    check_generation(generation);
    // the totals of this evaluation were formed for the cell volume: a volume
    // equal to it up to rounding rescales them instead of a second reduction
    if (reduced_ && std::isfinite(volume) && volume > 0.0 &&
        std::abs(volume - reduced_volume_) <= 1e-12 * reduced_volume_) {
        const double f = reduced_volume_ / volume;
        for (int q = 0; q < 9; ++q) out9[q] = volume == reduced_volume_ ? host_totals_[1 + q] : host_totals_[1 + q] * f;
        return;
    }
    reduce(volume);
    std::memcpy(out9, host_totals_ + 1, 9 * sizeof(double));
}

double Evaluator::total_energy(std::uint64_t generation)
{
    check_generation(generation);
    reduce(reduced_ ? reduced_volume_ : 1.0);
    return host_totals_[0];
}

}  // namespace sxl
