// Host-side model loading and compact radial tabulation (see model.hpp).
#include "model.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <fstream>
#include <map>
#include <set>
#include <sstream>
#include <stdexcept>

#include "json.hpp"

namespace sxl {
namespace json {

Value parse_file(const std::string& path)
{
    std::FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) throw std::invalid_argument("cannot open model file '" + path + "'");
    std::fseek(f, 0, SEEK_END);
    const long size = std::ftell(f);
    std::fseek(f, 0, SEEK_SET);
    std::string text(static_cast<std::size_t>(std::max(0L, size)), '\0');
    const std::size_t got = std::fread(text.data(), 1, text.size(), f);
    std::fclose(f);
    if (got != text.size()) throw std::invalid_argument("cannot read model file '" + path + "'");
    Parser parser(text.data(), text.data() + text.size());
    return parser.parse_document();
}

}  // namespace json

namespace {

using json::Value;

void require(bool ok, const std::string& message)
{
    if (!ok) throw std::invalid_argument(message);
}

std::vector<double> finite(std::vector<double> v, const std::string& what)
{
    for (double x : v)
        if (!std::isfinite(x) || std::abs(x) > 3.4028234663852886e38)
            throw std::invalid_argument(
                "MACE model contains a value outside the requested precision range (" + what + ").");
    return v;
}

std::vector<double> numbers(const Value& v, const std::string& what, std::size_t expected)
{
    std::vector<double> out = finite(v.flat_numbers(what), what);
    if (expected != static_cast<std::size_t>(-1) && out.size() != expected) {
        std::ostringstream os;
        os << what << " has " << out.size() << " values, expected " << expected;
        throw std::invalid_argument(os.str());
    }
    return out;
}

// Prediction-head selection (reference prediction_heads.hpp:10-89): a file
// with a prediction_heads section has its selected head's parameters copied
// over the top-level fields.
Value select_head(Value data, const std::string& requested, std::string& selected,
                  std::vector<std::string>& available)
{
    const Value* section = data.find("prediction_heads");
    if (!section) {
        const Value* h = data.find("head");
        const std::string legacy = h && h->kind == Value::Kind::string ? h->str : std::string();
        if (!requested.empty() && requested != legacy) {
            if (legacy.empty())
                throw std::invalid_argument(
                    "This JSON in the original Symmetrix format does not identify a prediction head.");
            throw std::invalid_argument("Requested prediction head '" + requested +
                                        "' is unavailable; the JSON contains '" + legacy + "'.");
        }
        selected = legacy;
        available.clear();
        if (!legacy.empty()) available.push_back(legacy);
        return data;
    }
    require(section->is_object() && section->contains("schema_version") &&
                section->at("schema_version").as_number() == 1,
            "prediction_heads has an unsupported schema version.");
    const Value& names_v = section->at("names");
    require(names_v.kind == Value::Kind::array, "prediction_heads.names must be an array.");
    std::vector<std::string> names;
    for (const auto& n : names_v.items) names.push_back(n.as_string("prediction head name"));
    std::set<std::string> unique(names.begin(), names.end());
    require(!names.empty() && unique.size() == names.size() && !unique.count(""),
            "prediction_heads.names must contain unique non-empty strings.");
    const Value& params = section->at("parameters");
    require(params.is_object() && params.size() == names.size(),
            "prediction_heads.parameters must define every named head.");
    // every head carries exactly the per-head fields of the format: atomic
    // energies, readout_1 (named after the H1 basis in format 4) and readout_2,
    // plus the ZBL coefficients when the model has ZBL
    std::set<std::string> expected = {"atomic_energies", "readout_2_weights_1", "readout_2_weights_2"};
    const Value* fv = data.find("symmetrix_format_version");
    const Value* mode = data.find("h1_affine_mode");
    const bool v4 = fv && fv->is_number() && fv->as_number() == 4;
    const bool pre = mode && mode->kind == Value::Kind::string && mode->str == "pre_linear_up";
    expected.insert(!v4 ? "readout_1_weights" : pre ? "readout_1_weights_for_H1_pre_linear_up"
                                                    : "readout_1_weights_for_M0");
    const Value* zbl = data.find("has_zbl");
    if (zbl && zbl->kind == Value::Kind::boolean && zbl->b) expected.insert("zbl_c");
    for (const auto& name : names) {
        const Value* head = params.find(name);
        require(head && head->is_object(), "prediction_heads.parameters must define every named head.");
        std::set<std::string> fields;
        for (const auto& kv : head->obj) fields.insert(kv.first);
        require(fields == expected, "Every prediction-head payload must contain exactly the supported fields.");
    }
    const Value* def = section->find("default");
    const std::string default_head = def && def->kind == Value::Kind::string ? def->str : "";
    require(unique.count(default_head) == 1, "prediction_heads.default must name a stored head.");
    selected = requested.empty() ? default_head : requested;
    require(unique.count(selected) == 1, "Requested prediction head '" + selected + "' is unavailable.");
    available = names;
    Value chosen = params.at(selected);
    for (auto& kv : chosen.obj) {
        bool replaced = false;
        for (auto& top : data.obj)
            if (top.first == kv.first) {
                top.second = kv.second;
                replaced = true;
            }
        if (!replaced) data.obj.emplace_back(kv.first, kv.second);
    }
    return data;
}

// Compact radial network (compact_radial.cpp:12-52, 172-194): SiLU MLP
// without biases; only the A0/A1 density networks carry the tanh-square
// postprocess.
RadialNetwork parse_network(const Value& def, const std::string& name, int inputs)
{
    RadialNetwork net;
    net.shape = def.at("shape").ints(name + " shape");
    const Value* post = def.find("postprocess");
    const std::string postprocess = post && post->kind == Value::Kind::string ? post->str : std::string();
    require(!post || post->kind == Value::Kind::string,
            "Compact radial network " + name + " has unsupported postprocessing.");
    require(postprocess.empty() || postprocess == "tanh-square",
            "Compact radial network " + name + " has unsupported postprocessing.");
    net.tanh_square = postprocess == "tanh-square";
    require(def.at("activation").as_string() == "silu",
            "Compact radial network " + name + " must use SiLU.");
    net.activation_scale = def.at("activation_scale").as_number();
    require(std::isfinite(net.activation_scale) && net.activation_scale > 0.0,
            "Compact radial network " + name + " has an invalid activation scale.");
    const Value& weights = def.at("weights");
    require(net.shape.size() >= 2 && weights.size() == net.shape.size() - 1,
            "Compact radial network " + name + " has an invalid shape.");
    require(net.shape.front() == inputs,
            "Compact radial network input does not match the Bessel basis.");
    for (std::size_t layer = 0; layer + 1 < net.shape.size(); ++layer) {
        require(net.shape[layer] > 0 && net.shape[layer + 1] > 0,
                "Compact radial network " + name + " has a non-positive layer size.");
        const std::size_t expected =
            static_cast<std::size_t>(net.shape[layer]) * net.shape[layer + 1];
        net.weights.push_back(numbers(weights[layer], name + " weights", expected));
    }
    return net;
}

// Monomials of one polynomial output.  A monomial listed again (the same
// index vector, in the same order) keeps the coefficient of its first entry:
// the reference stores an output's terms in a std::map keyed by the index
// vector, whose insert ignores later duplicates
// (libsymmetrix/source/multivariate_polynomial.cpp:36-46; the Kokkos loader
// does the same, mace_kokkos_model.cpp:55-76).  Permutations of one vector
// ([0,1] and [1,0]) are distinct keys there and stay distinct terms here.
// keep[j] tells whether JSON entry j is a term; degree and index receive the
// kept terms, indices sorted ascending (the product does not depend on their
// order).
void parse_monomials(const Value& list, const std::string& what, std::vector<int>& degree,
                     std::vector<int>& index, int num_variables, std::vector<char>& keep)
{
    require(list.kind == Value::Kind::array || (list.kind == Value::Kind::numbers && list.nums.empty()),
            what + " must be a list of monomials");
    std::set<std::vector<int>> seen;
    keep.clear();
    for (const auto& mono : list.items) {
        std::vector<int> m = mono.ints(what);
        require(!m.empty() && m.size() <= 3,
                what + ": only monomials of degree 1 to 3 (correlation <= 3) are supported");
        const bool first = seen.insert(m).second;
        keep.push_back(first ? 1 : 0);
        if (!first) continue;
        std::sort(m.begin(), m.end());
        for (int v : m) require(v >= 0 && v < num_variables, what + " references an invalid input");
        degree.push_back(static_cast<int>(m.size()));
        index.push_back(m[0]);
        index.push_back(m.size() > 1 ? m[1] : 0);
        index.push_back(m.size() > 2 ? m[2] : 0);
    }
}

}  // namespace

HostModel HostModel::load(const std::string& path, const std::string& head)
{
    HostModel m;
    Value file = select_head(json::parse_file(path), head, m.selected_head, m.available_heads);

    const Value* mt = file.find("model_type");
    const std::string model_type = mt ? mt->as_string() : "MACE";
    if (model_type == "MACE_Nonlinear")
        throw std::invalid_argument(
            "MACE_Nonlinear JSON is a different model family; this evaluator loads standard MACE.");
    require(model_type == "MACE", "Format version 4 is the standard MACE / MACEField format.");

    m.num_elements = file.at("num_elements").as_int("num_elements");
    m.channels = file.at("num_channels").as_int("num_channels");
    const Value* ni = file.find("num_interactions");
    const int num_interactions = ni ? ni->as_int() : 2;
    const Value* slr = file.find("single_layer_readout");
    require(!(slr && slr->as_bool()) && num_interactions == 2,
            "Only two-interaction MACE models are supported by this evaluator.");
    m.r_cut = file.at("r_cut").as_number("r_cut");
    m.l_max = file.at("l_max").as_int("l_max");
    m.L_max = file.at("L_max").as_int("L_max");
    require(m.num_elements > 0 && m.channels > 0 && m.channels <= 1024,
            "MACE model has invalid element or channel counts.");
    require(m.l_max >= 0 && m.l_max <= 3 && m.L_max >= 0 && m.L_max <= m.l_max,
            "MACE model requires 0 <= L_max <= l_max <= 3.");
    require(std::isfinite(m.r_cut) && m.r_cut > 0.0, "MACE model has an invalid r_cut.");
    m.num_lm = (m.l_max + 1) * (m.l_max + 1);
    m.num_LM = (m.L_max + 1) * (m.L_max + 1);
    const int ne = m.num_elements, C = m.channels;
    m.atomic_numbers = file.at("atomic_numbers").ints("atomic_numbers");
    m.atomic_energies = numbers(file.at("atomic_energies"), "atomic_energies", ne);
    require(static_cast<int>(m.atomic_numbers.size()) == ne,
            "atomic_numbers does not match num_elements.");

    // ZBL (mace_kokkos_model.cpp:190-198, zbl_kokkos.cpp:12-56)
    m.has_zbl = file.at("has_zbl").as_bool("has_zbl");
    if (m.has_zbl) {
        m.zbl_a_exp = file.at("zbl_a_exp").as_number("zbl_a_exp");
        m.zbl_a_prefactor = file.at("zbl_a_prefactor").as_number("zbl_a_prefactor");
        const std::vector<double> c = numbers(file.at("zbl_c"), "zbl_c", static_cast<std::size_t>(-1));
        require(c.size() == 4, "ZBL requires four screening coefficients");
        for (int q = 0; q < 4; ++q) m.zbl_c[q] = c[q];
        m.zbl_radii = numbers(file.at("zbl_covalent_radii"), "zbl_covalent_radii", static_cast<std::size_t>(-1));
        require(!m.zbl_radii.empty(), "ZBL requires at least one covalent radius");
        require(m.zbl_a_prefactor > 0.0, "ZBL screening prefactor must be positive");
        m.zbl_p = file.at("zbl_p").as_int("zbl_p");
        require(m.zbl_p >= 1, "ZBL envelope power must be positive");
        require(std::isfinite(m.zbl_a_exp), "ZBL has an invalid screening exponent");
        for (int z : m.atomic_numbers)
            require(z >= 0 && z < static_cast<int>(m.zbl_radii.size()),
                    "ZBL covalent radii do not cover the model's atomic numbers");
    }
    const Value* hf = file.find("has_field_coupling");
    require(!(hf && hf->as_bool()), "MACEField coupling is not supported.");
    const Value* fr = file.find("first_interaction_residual");
    m.first_residual = fr && fr->as_bool();

    // format 4, m0_composite or pre_linear_up basis (h1_affine_schema.hpp:168-258)
    const Value* fv = file.find("symmetrix_format_version");
    const int version = fv ? fv->as_int() : 1;
    require(version == 4,
            "Only Symmetrix MACE JSON format version 4 is supported; re-export older files.");
    const Value* mode = file.find("h1_affine_mode");
    require(mode && mode->kind == Value::Kind::string &&
                (mode->str == "m0_composite" || mode->str == "pre_linear_up"),
            "Symmetrix MACE format version 4 requires h1_affine_mode 'm0_composite' or "
            "'pre_linear_up'.");
    m.pre_linear_up = mode->str == "pre_linear_up";
    const Value* av = file.find("h1_affine_version");
    require(av && av->as_number() == 1, "Unsupported h1_affine_version (supported: 1).");
    require(!file.contains("readout_1_weights") && !file.contains("H2_weights_for_H1"),
            "A format-version-4 MACE JSON must not contain the old-basis readout_1_weights or "
            "H2_weights_for_H1 fields.");
    const char* readout_key =
        m.pre_linear_up ? "readout_1_weights_for_H1_pre_linear_up" : "readout_1_weights_for_M0";
    const char* skip_key = m.pre_linear_up ? "H2_weights_for_H1_pre_linear_up" : "H2_weights_for_M0";
    if (m.pre_linear_up)
        require(!file.contains("readout_1_weights_for_M0") && !file.contains("H2_weights_for_M0"),
                "A 'pre_linear_up' MACE JSON must not contain readout_1_weights_for_M0 or "
                "H2_weights_for_M0.");
    else
        require(!file.contains("readout_1_weights_for_H1_pre_linear_up") &&
                    !file.contains("H2_weights_for_H1_pre_linear_up"),
                "A 'm0_composite' MACE JSON must not contain readout_1_weights_for_H1_pre_linear_up "
                "or H2_weights_for_H1_pre_linear_up.");
    require(m.pre_linear_up || !m.first_residual,
            "The m0_composite basis cannot represent first-interaction residual or field-coupled "
            "features; such models use h1_affine_mode 'pre_linear_up'.");
    require(!m.pre_linear_up || file.contains("H1_product_weights"),
            "The pre_linear_up basis requires H1_product_weights.");
    require(file.contains(readout_key) && file.contains(skip_key),
            std::string("A '") + mode->str + "' MACE JSON requires " + readout_key + " and " + skip_key + ".");

    // compact radial model (compact_radial.cpp:110-205)
    const Value* rr = file.find("radial_representation");
    require(rr && rr->kind == Value::Kind::string && rr->str == "compact",
            "Only the compact radial representation is supported.");
    const Value& cr = file.at("compact_radial");
    m.grid_min = cr.at("spline_grid_min").as_number();
    m.spline_points = cr.at("num_spline_points").as_int();
    require(std::isfinite(m.grid_min) && m.grid_min > 0.0,
            "Compact radial model has an invalid spline grid minimum.");
    require(m.spline_points >= 4, "Compact radial model requires at least four spline points.");
    m.spline_h = (m.r_cut - m.grid_min) / (m.spline_points - 1);
    require(m.spline_h > 0.0, "Compact radial model has an invalid spline grid.");
    const Value& basis = cr.at("basis");
    require(basis.at("type").as_string() == "bessel",
            "Compact radial model only supports a Bessel basis.");
    m.bessel_weights = numbers(basis.at("weights"), "Bessel weights", static_cast<std::size_t>(-1));
    m.bessel_prefactor = basis.at("prefactor").as_number();
    require(!m.bessel_weights.empty() && std::isfinite(m.bessel_prefactor),
            "Compact radial model has invalid Bessel data.");
    const Value& cut = cr.at("cutoff");
    require(cut.at("type").as_string() == "polynomial",
            "Compact radial model only supports a polynomial cutoff.");
    m.cutoff_rmax = cut.at("r_max").as_number();
    m.cutoff_p = cut.at("p").as_int();
    require(std::isfinite(m.cutoff_rmax) && m.cutoff_p > 0,
            "Compact radial model has invalid cutoff data.");
    require(std::abs(m.cutoff_rmax - m.r_cut) <= 1e-12,
            "Compact radial cutoff does not match model r_cut.");
    const Value& transform = cr.at("distance_transform");
    const std::string transform_type = transform.at("type").as_string();
    m.agnesi = transform_type == "agnesi";
    if (m.agnesi) {
        m.agnesi_a = transform.at("a").as_number();
        m.agnesi_q = transform.at("q").as_number();
        m.agnesi_p = transform.at("p").as_number();
        m.agnesi_radii = numbers(transform.at("covalent_radii"), "covalent_radii", static_cast<std::size_t>(-1));
        require(static_cast<int>(m.agnesi_radii.size()) == ne,
                "Compact radial covalent radii do not match atomic numbers.");
        bool ok = std::isfinite(m.agnesi_a) && std::isfinite(m.agnesi_q) && std::isfinite(m.agnesi_p);
        for (double v : m.agnesi_radii) ok = ok && std::isfinite(v) && v > 0.0;
        require(ok, "Compact radial model has invalid Agnesi data.");
    } else {
        require(transform_type == "none", "Compact radial model has an unsupported distance transform.");
    }
    const Value& nets = cr.at("networks");
    const int nb = static_cast<int>(m.bessel_weights.size());
    m.R0 = parse_network(nets.at("R0"), "R0", nb);
    require(nets.contains("R1"), "Compact radial R1 network does not match the MACE interaction count.");
    m.R1 = parse_network(nets.at("R1"), "R1", nb);
    require(!m.R0.tanh_square && !m.R1.tanh_square, "Compact radial R0/R1 networks cannot use postprocessing.");
    auto density_network = [&](const char* name, RadialNetwork& net) {
        net = parse_network(nets.at(name), name, nb);
        require(net.shape.back() == 1 && net.tanh_square,
                std::string("Compact radial ") + name + " network has an invalid shape or postprocessing.");
    };
    const Value* a0s = file.find("A0_scaled");
    const Value* a1s = file.find("A1_scaled");
    require(a0s != nullptr, "MACE model is missing A0_scaled.");
    m.A0_scaled = a0s->as_bool();
    m.A1_scaled = a1s && a1s->as_bool();
    require(m.A0_scaled == nets.contains("A0"), "Compact radial A0 network does not match A0_scaled.");
    require(m.A1_scaled == nets.contains("A1"), "Compact radial A1 network does not match A1_scaled.");
    if (m.A0_scaled) density_network("A0", m.A0net);
    if (m.A1_scaled) density_network("A1", m.A1net);

    require(m.R0.shape.back() == (m.l_max + 1) * C, "Compact radial R0 output has an invalid size.");

    m.H0 = numbers(file.at("H0_weights"), "H0_weights", static_cast<std::size_t>(ne) * C);
    m.A0W = numbers(file.at("A0_weights"), "A0_weights",
                    static_cast<std::size_t>(ne) * (m.l_max + 1) * C * C);

    // M0 symmetric contraction
    const Value& m0_mono = file.at("M0_monomials");
    const Value& m0_w = file.at("M0_weights");
    m.m0_offsets.push_back(0);
    std::vector<std::vector<char>> m0_keep(m.num_LM);
    for (int LM = 0; LM < m.num_LM; ++LM) {
        const std::string key = std::to_string(LM);
        std::vector<int> deg, idx;
        parse_monomials(m0_mono.at(key), "M0_monomials", deg, idx, m.num_lm, m0_keep[LM]);
        m.m0_degree.insert(m.m0_degree.end(), deg.begin(), deg.end());
        m.m0_index.insert(m.m0_index.end(), idx.begin(), idx.end());
        m.m0_offsets.push_back(m.m0_offsets.back() + static_cast<int>(deg.size()));
    }
    const int T0 = m.m0_offsets.back();
    m.m0_coef.assign(static_cast<std::size_t>(ne) * T0 * C, 0.0);
    for (int a = 0; a < ne; ++a) {
        const Value& wa = m0_w.at(std::to_string(a));
        for (int LM = 0; LM < m.num_LM; ++LM) {
            const Value& wl = wa.at(std::to_string(LM));
            const std::vector<char>& keep = m0_keep[LM];
            for (int k = 0; k < C; ++k) {
                std::vector<double> c = numbers(wl.at(std::to_string(k)), "M0_weights", keep.size());
                for (std::size_t j = 0, t = 0; j < keep.size(); ++j)
                    if (keep[j]) m.m0_coef[(static_cast<std::size_t>(a) * T0 + m.m0_offsets[LM] + t++) * C + k] = c[j];
            }
        }
    }

    const std::size_t h1_size = static_cast<std::size_t>(m.L_max + 1) * C * C;
    m.H1W = numbers(file.at("H1_weights"), "H1_weights", h1_size);

    // split H1 weights and the first-interaction residual (mace.cpp:2790-2829)
    auto optional_numbers = [&](const char* key) {
        const Value* v = file.find(key);
        return v ? numbers(*v, key, static_cast<std::size_t>(-1)) : std::vector<double>{};
    };
    const std::vector<double> product = optional_numbers("H1_product_weights");
    const std::vector<double> linear_up = optional_numbers("H1_linear_up_weights");
    const std::vector<double> residual = optional_numbers("H1_first_residual_weights");
    const std::size_t residual_size = static_cast<std::size_t>(ne) * m.num_LM * C;
    if (m.first_residual) {
        require(residual.size() == residual_size, "Residual-first MACE JSON has an invalid H1 residual extent.");
        require(product.size() == h1_size && linear_up.size() == h1_size,
                "Residual-first MACE JSON requires split H1 weights.");
        m.residual = residual;
        // fused residual: residual U, per element, per l block
        m.residual_fused.assign(residual_size, 0.0);
        for (int a = 0; a < ne; ++a)
            for (int l = 0; l <= m.L_max; ++l)
                for (int lm = l * l; lm < (l + 1) * (l + 1); ++lm) {
                    const double* res = residual.data() + (static_cast<std::size_t>(a) * m.num_LM + lm) * C;
                    double* out = m.residual_fused.data() + (static_cast<std::size_t>(a) * m.num_LM + lm) * C;
                    for (int in = 0; in < C; ++in) {
                        const double* u = linear_up.data() + (static_cast<std::size_t>(l) * C + in) * C;
                        for (int k = 0; k < C; ++k) out[k] += res[in] * u[k];
                    }
                }
    } else {
        require(residual.empty(), "Non-residual MACE JSON must not contain H1 residual weights.");
    }
    if (m.pre_linear_up) {
        require(product.size() == h1_size,
                "The pre_linear_up basis requires H1_product_weights of the H1_weights extent.");
        m.H1P = product;
    }

    // second interaction tables
    m.Phi1_l = file.at("Phi1_l").ints("Phi1_l");
    m.Phi1_l1 = file.at("Phi1_l1").ints("Phi1_l1");
    m.Phi1_l2 = file.at("Phi1_l2").ints("Phi1_l2");
    m.Phi1_lme = file.at("Phi1_lme").ints("Phi1_lme");
    m.Phi1_row = file.at("Phi1_lelm1lm2").ints("Phi1_lelm1lm2");
    m.Phi1_cg = numbers(file.at("Phi1_clebsch_gordan"), "Phi1_clebsch_gordan", m.Phi1_lme.size());
    require(m.Phi1_l.size() == m.Phi1_l1.size() && m.Phi1_l.size() == m.Phi1_l2.size() &&
                m.Phi1_row.size() == m.Phi1_lme.size(),
            "Phi1 path and term tables have inconsistent lengths.");
    require(m.R1.shape.back() == m.num_paths() * C, "Compact radial R1 output has an invalid size.");
    std::vector<int> num_e(m.l_max + 1, 0);
    for (int l : m.Phi1_l) {
        require(l >= 0 && l <= m.l_max, "Phi1_l holds an invalid output l.");
        num_e[l] += 1;
    }
    const Value& a1 = file.at("A1_weights");
    require(static_cast<int>(a1.size()) == m.l_max + 1, "A1_weights must hold one matrix per l.");
    for (int l = 0; l <= m.l_max; ++l)
        m.A1W.push_back(numbers(a1[l], "A1_weights", static_cast<std::size_t>(num_e[l]) * C * C));

    // M1
    std::vector<int> deg1, idx1;
    std::vector<char> m1_keep;
    parse_monomials(file.at("M1_monomials"), "M1_monomials", deg1, idx1, m.num_lm, m1_keep);
    m.m1_degree = deg1;
    m.m1_index = idx1;
    const int T1 = static_cast<int>(deg1.size());
    m.m1_coef.assign(static_cast<std::size_t>(ne) * T1 * C, 0.0);
    const Value& m1_w = file.at("M1_weights");
    for (int a = 0; a < ne; ++a) {
        const Value& wa = m1_w.at(std::to_string(a));
        for (int k = 0; k < C; ++k) {
            std::vector<double> c = numbers(wa.at(std::to_string(k)), "M1_weights", m1_keep.size());
            for (std::size_t j = 0, t = 0; j < m1_keep.size(); ++j)
                if (m1_keep[j]) m.m1_coef[(static_cast<std::size_t>(a) * T1 + t++) * C + k] = c[j];
        }
    }

    // H2 and readouts: skip map and readout_1 on the scalar x of the basis
    const Value& skip = file.at(skip_key);
    require(skip.kind == Value::Kind::array && static_cast<int>(skip.size()) == ne,
            std::string(skip_key) + " must hold one row per element.");
    for (std::size_t a = 0; a < skip.size(); ++a)
        require(skip[a].is_array() && skip[a].size() == static_cast<std::size_t>(C) * C,
                std::string("Every ") + skip_key + " row must hold num_channels^2 values.");
    m.H2M0 = numbers(skip, skip_key, static_cast<std::size_t>(ne) * C * C);
    m.H2M1 = numbers(file.at("H2_weights_for_M1"), "H2_weights_for_M1",
                     static_cast<std::size_t>(C) * C);
    const Value& readout = file.at(readout_key);
    require(readout.is_array() && readout.size() == static_cast<std::size_t>(C),
            std::string(readout_key) + " must hold num_channels values.");
    m.readout_q = numbers(readout, readout_key, C);
    const Value* hs = file.find("readout_2_hidden_size");
    m.readout_hidden = hs ? hs->as_int() : 16;
    require(m.readout_hidden > 0 && m.readout_hidden <= 64,
            "MACE nonlinear readout weights do not match the declared hidden size.");
    m.readout_w1 = numbers(file.at("readout_2_weights_1"), "readout_2_weights_1",
                           static_cast<std::size_t>(m.readout_hidden) * C);
    m.readout_w2 = numbers(file.at("readout_2_weights_2"), "readout_2_weights_2",
                           static_cast<std::size_t>(m.readout_hidden));
    m.readout_scale = file.at("readout_2_scale_factor").as_number();
    return m;
}

// Compact radial tabulation (compact_radial.cpp:227-370): Bessel features with
// the polynomial cutoff on the knots (of the Agnesi-transformed distance when
// the model has that transform), the SiLU MLP (tanh(y^2) on the output of a
// density network), and knot derivatives from the tridiagonal rule with a
// not-a-knot-like left end and a zero derivative at r_cut.
void HostModel::radial_tables(const RadialNetwork& net, int type_i, int type_j,
                              std::vector<double>& values, std::vector<double>& derivs) const
{
    if (type_i < 0 || type_i >= num_elements || type_j < 0 || type_j >= num_elements)
        throw std::out_of_range("Compact radial model type index is out of range.");
    const int P = spline_points;
    const int nb = static_cast<int>(bessel_weights.size());
    std::vector<double> layer(static_cast<std::size_t>(P) * nb);
    const double r0 = agnesi ? 0.5 * (agnesi_radii[type_i] + agnesi_radii[type_j]) : 1.0;
    for (int node = 0; node < P; ++node) {
        const double r = grid_min + node * spline_h;
        double t = r;
        if (agnesi) {
            const double s = r / r0;
            t = 1.0 / (1.0 + agnesi_a * std::pow(s, agnesi_q) / (1.0 + std::pow(s, agnesi_q - agnesi_p)));
        }
        double cutoff_value = 0.0;
        if (r < cutoff_rmax) {
            const double s = r / cutoff_rmax;
            const double p = cutoff_p;
            cutoff_value = 1.0 - ((p + 1.0) * (p + 2.0) / 2.0) * std::pow(s, p) +
                           p * (p + 2.0) * std::pow(s, p + 1) -
                           (p * (p + 1.0) / 2.0) * std::pow(s, p + 2);
        }
        for (int b = 0; b < nb; ++b)
            layer[static_cast<std::size_t>(node) * nb + b] =
                bessel_prefactor * std::sin(bessel_weights[b] * t) / t * cutoff_value;
    }
    int width = nb;
    for (std::size_t l = 0; l < net.weights.size(); ++l) {
        const int out = net.shape[l + 1];
        const std::vector<double>& W = net.weights[l];
        std::vector<double> next(static_cast<std::size_t>(P) * out, 0.0);
        for (int node = 0; node < P; ++node) {
            const double* x = layer.data() + static_cast<std::size_t>(node) * width;
            double* y = next.data() + static_cast<std::size_t>(node) * out;
            for (int o = 0; o < out; ++o) {
                const double* w = W.data() + static_cast<std::size_t>(o) * width;
                double acc = 0.0;
                for (int i = 0; i < width; ++i) acc += w[i] * x[i];
                y[o] = acc;
            }
            if (l + 1 < net.weights.size())
                for (int o = 0; o < out; ++o)
                    y[o] = net.activation_scale * y[o] / (1.0 + std::exp(-y[o]));
        }
        layer.swap(next);
        width = out;
    }
    const int F = width;
    if (net.tanh_square)
        for (double& v : layer) v = std::tanh(v * v);
    values.assign(static_cast<std::size_t>(F) * P, 0.0);
    derivs.assign(static_cast<std::size_t>(F) * P, 0.0);
    const int U = P - 2;
    const double h = spline_h;
    std::vector<double> lower(U, 0.0), diag(U, 4.0), upper(U, 0.0), rhs(U), sol(U);
    for (int f = 0; f < F; ++f) {
        double* v = values.data() + static_cast<std::size_t>(f) * P;
        for (int node = 0; node < P; ++node) v[node] = layer[static_cast<std::size_t>(node) * F + f];
        std::fill(lower.begin(), lower.end(), 0.0);
        std::fill(diag.begin(), diag.end(), 4.0);
        std::fill(upper.begin(), upper.end(), 0.0);
        const double left = 2.0 * (-v[0] + 2.0 * v[1] - v[2]) / h;
        upper[0] = 2.0;
        rhs[0] = 3.0 * (v[2] - v[0]) / h - left;
        for (int node = 2; node < P - 1; ++node) {
            const int row = node - 1;
            lower[row] = 1.0;
            if (node + 1 <= P - 2) upper[row] = 1.0;
            rhs[row] = 3.0 * (v[node + 1] - v[node - 1]) / h;
        }
        for (int row = 1; row < U; ++row) {
            const double factor = lower[row] / diag[row - 1];
            diag[row] -= factor * upper[row - 1];
            rhs[row] -= factor * rhs[row - 1];
        }
        sol[U - 1] = rhs[U - 1] / diag[U - 1];
        for (int row = U - 2; row >= 0; --row) sol[row] = (rhs[row] - upper[row] * sol[row + 1]) / diag[row];
        double* d = derivs.data() + static_cast<std::size_t>(f) * P;
        for (int node = 1; node < P - 1; ++node) d[node] = sol[node - 1];
        d[0] = d[2] + left;
        d[P - 1] = 0.0;
    }
}

}  // namespace sxl
