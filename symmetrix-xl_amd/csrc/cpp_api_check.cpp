// Drives the C++ facade (include/symmetrix_amd.hpp) end to end for the tests.
//
//   cpp_api_check MODEL HEAD IN OUT
//
// IN (native byte order): int32 n, int32 types[n], f64 positions[3n],
// f64 cell[9], f64 inverse_cell[9], f64 cutoff, f64 volume.
// OUT: f64 total_energy, f64 node_energies[n], f64 atom_forces[3n],
// f64 stress[9], int64 num_edges, f64 directed_forces[3 num_edges].
// stdout: one line "r_cut l_max L_max num_channels num_elements selected_head
// heads...".  An exception is reported on stderr as "<kind>: <message>" with
// exit status 3; a usage or file error exits with status 2.
#include <cstdint>
#include <cstdio>
#include <exception>
#include <fstream>
#include <iostream>
#include <stdexcept>
#include <string>
#include <vector>

#include "symmetrix_amd.hpp"

namespace {

template <class T>
bool read_values(std::ifstream& in, std::vector<T>& v, std::size_t n)
{
    v.resize(n);
    in.read(reinterpret_cast<char*>(v.data()), static_cast<std::streamsize>(n * sizeof(T)));
    return static_cast<bool>(in);
}

template <class T>
void write_values(std::ofstream& out, const T* v, std::size_t n)
{
    out.write(reinterpret_cast<const char*>(v), static_cast<std::streamsize>(n * sizeof(T)));
}

int run(const std::string& model, const std::string& head, const std::string& in_path, const std::string& out_path)
{
    std::ifstream in(in_path, std::ios::binary);
    std::int32_t n = 0;
    in.read(reinterpret_cast<char*>(&n), sizeof(n));
    std::vector<int> types;
    std::vector<double> positions, cell, inverse_cell, scalars;
    if (!in || n < 0 || !read_values(in, types, static_cast<std::size_t>(n)) ||
        !read_values(in, positions, 3 * static_cast<std::size_t>(n)) || !read_values(in, cell, 9) ||
        !read_values(in, inverse_cell, 9) || !read_values(in, scalars, 2)) {
        std::cerr << "input: cannot read " << in_path << "\n";
        return 2;
    }
    const double cutoff = scalars[0], volume = scalars[1];

    symmetrix_amd::MACEKokkosFloat ev(model, head);
    std::cout << ev.r_cut << " " << ev.l_max << " " << ev.L_max << " " << ev.num_channels << " "
              << ev.atomic_numbers_host.size() << " " << (ev.selected_head.empty() ? "-" : ev.selected_head);
    for (const std::string& h : ev.available_heads) std::cout << " " << h;
    std::cout << "\n";

    const auto [generation, num_edges] = ev.prepare_periodic_factorized_graph(types, positions, cell, inverse_cell,
                                                                              cutoff);
    ev.compute_prepared_factorized_positions(generation, positions);
    ev.reduce_prepared_node_forces(generation);
    ev.reduce_prepared_stress(volume, generation);
    const double energy = ev.total_energy(generation);
    const std::vector<double>& energies = ev.node_energies();
    const std::vector<double>& directed = ev.node_forces();
    // the workspace report names the prepared graph
    if (ev.workspace_json().find("\"graph_generation\": " + std::to_string(generation)) == std::string::npos) {
        std::cerr << "workspace_json: generation " << generation << " missing\n";
        return 3;
    }

    std::ofstream out(out_path, std::ios::binary);
    write_values(out, &energy, 1);
    write_values(out, energies.data(), energies.size());
    write_values(out, ev.atom_forces().data(), ev.atom_forces().size());
    write_values(out, ev.stress_tensor().data(), ev.stress_tensor().size());
    const std::int64_t edges = static_cast<std::int64_t>(num_edges);
    write_values(out, &edges, 1);
    write_values(out, directed.data(), directed.size());
    if (!out) {
        std::cerr << "output: cannot write " << out_path << "\n";
        return 2;
    }
    return 0;
}

}  // namespace

int main(int argc, char** argv)
{
    if (argc != 5) {
        std::cerr << "usage: cpp_api_check MODEL HEAD IN OUT\n";
        return 2;
    }
    try {
        return run(argv[1], argv[2], argv[3], argv[4]);
    } catch (const std::invalid_argument& e) {
        std::cerr << "invalid_argument: " << e.what() << "\n";
    } catch (const std::out_of_range& e) {
        std::cerr << "out_of_range: " << e.what() << "\n";
    } catch (const std::length_error& e) {
        std::cerr << "length_error: " << e.what() << "\n";
    } catch (const std::logic_error& e) {
        std::cerr << "logic_error: " << e.what() << "\n";
    } catch (const std::runtime_error& e) {
        std::cerr << "runtime_error: " << e.what() << "\n";
    } catch (const std::exception& e) {
        std::cerr << "exception: " << e.what() << "\n";
    }
    return 3;
}
