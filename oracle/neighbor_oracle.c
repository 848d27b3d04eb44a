/*
 * TEST INFRASTRUCTURE ONLY -- the CPU oracle for the periodic neighbour graph.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this code, and only as the checker.  The product never calls it.
 *
 * Serial restatement of the reference's cell-binned periodic neighbour graph
 * (libsymmetrix/source/neighbor_graph_kokkos.cpp:38-405):
 *   wrap to fractional [0,1) and record the wrap shifts        (:117-141)
 *   bins per axis = max(1, floor(face_height / cutoff)),
 *   stencil reach = ceil(cutoff*|inv column|*bins) + 1          (:143-166)
 *   count -> scan -> fill -> ascending sort within each bin     (:182-249)
 *   per receiver: dz, dy, dx stencil order, bin atoms ascending,
 *   skip self at zero image, keep d^2 <= cutoff^2               (:258-332)
 *   shifts = image - wrap(source) + wrap(receiver)               (:312-316)
 *   fractional_xyz = wrapped_frac(source) - wrapped_frac(recv) + image
 * Double-precision arithmetic is kept in the same operation order with no
 * contraction (the Makefile passes -ffp-contract=off), so the edge list is
 * bit-identical to a device build that follows the same order.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define NB_OK 0
#define NB_INVALID_ARGUMENT 1
#define NB_LENGTH_ERROR 2
#define NB_ALLOC_ERROR 3

static const char* nb_last_error = "";

const char* oracle_neighbor_last_error(void) { return nb_last_error; }

static int floor_div(int numerator, int denominator)
{
    const int quotient = numerator / denominator;
    const int remainder = numerator % denominator;
    return quotient - ((remainder != 0 && remainder < 0) ? 1 : 0);
}

typedef struct {
    int num_nodes;
    int bins[3];
    int reach[3];
    double cell[9];
    double cutoff_squared;
    double* wrapped_positions;   /* N x 3 */
    double* wrapped_fractional;  /* N x 3 */
    int* wrap_shifts;            /* N x 3 */
    int* atom_bins;              /* N */
    int* bin_offsets;            /* bins + 1 */
    int* bin_atoms;              /* N */
} nb_state;

static void nb_free(nb_state* s)
{
    free(s->wrapped_positions);
    free(s->wrapped_fractional);
    free(s->wrap_shifts);
    free(s->atom_bins);
    free(s->bin_offsets);
    free(s->bin_atoms);
    memset(s, 0, sizeof(*s));
}

static int nb_prepare(nb_state* s, const double* positions, int num_nodes,
                      const double* cell, const double* inverse_cell, double cutoff)
{
    memset(s, 0, sizeof(*s));
    if (!isfinite(cutoff) || !(cutoff > 0.0)) {
        nb_last_error = "neighbor graph cutoff must be finite and positive";
        return NB_INVALID_ARGUMENT;
    }
    if (num_nodes < 0) {
        nb_last_error = "neighbor graph input extents are inconsistent";
        return NB_INVALID_ARGUMENT;
    }
    for (int i = 0; i < 3 * num_nodes; ++i)
        if (!isfinite(positions[i])) {
            nb_last_error = "neighbor graph positions must be finite";
            return NB_INVALID_ARGUMENT;
        }
    for (int i = 0; i < 9; ++i)
        if (!isfinite(cell[i]) || !isfinite(inverse_cell[i])) {
            nb_last_error = "neighbor graph cell must be finite";
            return NB_INVALID_ARGUMENT;
        }
    for (int row = 0; row < 3; ++row)
        for (int column = 0; column < 3; ++column) {
            double product = 0.0;
            for (int inner = 0; inner < 3; ++inner)
                product += cell[3 * row + inner] * inverse_cell[3 * inner + column];
            const double expected = row == column ? 1.0 : 0.0;
            if (fabs(product - expected) > 1e-9) {
                nb_last_error = "neighbor graph cell and inverse cell are inconsistent";
                return NB_INVALID_ARGUMENT;
            }
        }
    s->num_nodes = num_nodes;
    memcpy(s->cell, cell, sizeof(s->cell));
    s->cutoff_squared = cutoff * cutoff;
    const size_t n = (size_t)num_nodes;
    s->wrapped_positions = (double*)malloc(sizeof(double) * 3 * (n + 1));
    s->wrapped_fractional = (double*)malloc(sizeof(double) * 3 * (n + 1));
    s->wrap_shifts = (int*)malloc(sizeof(int) * 3 * (n + 1));
    s->atom_bins = (int*)malloc(sizeof(int) * (n + 1));
    s->bin_atoms = (int*)malloc(sizeof(int) * (n + 1));
    if (!s->wrapped_positions || !s->wrapped_fractional || !s->wrap_shifts
        || !s->atom_bins || !s->bin_atoms) {
        nb_free(s);
        nb_last_error = "neighbor graph allocation failed";
        return NB_ALLOC_ERROR;
    }
    for (int atom = 0; atom < num_nodes; ++atom) {
        double fractional[3];
        for (int axis = 0; axis < 3; ++axis) {
            double value = 0.0;
            for (int component = 0; component < 3; ++component)
                value += positions[3 * atom + component] * inverse_cell[3 * component + axis];
            const int wrap = (int)floor(value);
            value -= wrap;
            fractional[axis] = value;
            s->wrapped_fractional[3 * atom + axis] = value;
            s->wrap_shifts[3 * atom + axis] = wrap;
        }
        for (int component = 0; component < 3; ++component) {
            double value = 0.0;
            for (int axis = 0; axis < 3; ++axis)
                value += fractional[axis] * cell[3 * axis + component];
            s->wrapped_positions[3 * atom + component] = value;
        }
    }
    for (int axis = 0; axis < 3; ++axis) {
        double inverse_norm_squared = 0.0;
        for (int component = 0; component < 3; ++component) {
            const double value = inverse_cell[3 * component + axis];
            inverse_norm_squared += value * value;
        }
        if (!(inverse_norm_squared > 0.0)) {
            nb_free(s);
            nb_last_error = "neighbor graph cell must be invertible";
            return NB_INVALID_ARGUMENT;
        }
        const double face_height = 1.0 / sqrt(inverse_norm_squared);
        const double bins = floor(face_height / cutoff);
        if (bins >= 2147483647.0) {
            nb_free(s);
            nb_last_error = "neighbor graph bin extent exceeds 32-bit indexing";
            return NB_LENGTH_ERROR;
        }
        s->bins[axis] = bins < 1.0 ? 1 : (int)bins;
        const double reach = ceil(cutoff * sqrt(inverse_norm_squared) * s->bins[axis]) + 1.0;
        if (reach >= 1073741823.0) {
            nb_free(s);
            nb_last_error = "neighbor graph stencil exceeds 32-bit indexing";
            return NB_LENGTH_ERROR;
        }
        s->reach[axis] = reach < 1.0 ? 1 : (int)reach;
    }
    const size_t num_bins_size = (size_t)s->bins[0] * (size_t)s->bins[1] * (size_t)s->bins[2];
    if (num_bins_size >= 2147483647u) {
        nb_free(s);
        nb_last_error = "neighbor graph bin count exceeds 32-bit indexing";
        return NB_LENGTH_ERROR;
    }
    const int num_bins = (int)num_bins_size;
    int* bin_sizes = (int*)calloc((size_t)num_bins + 1, sizeof(int));
    s->bin_offsets = (int*)malloc(sizeof(int) * ((size_t)num_bins + 1));
    if (!bin_sizes || !s->bin_offsets) {
        free(bin_sizes);
        nb_free(s);
        nb_last_error = "neighbor graph allocation failed";
        return NB_ALLOC_ERROR;
    }
    for (int atom = 0; atom < num_nodes; ++atom) {
        int x = (int)(s->wrapped_fractional[3 * atom + 0] * s->bins[0]);
        int y = (int)(s->wrapped_fractional[3 * atom + 1] * s->bins[1]);
        int z = (int)(s->wrapped_fractional[3 * atom + 2] * s->bins[2]);
        if (x > s->bins[0] - 1) x = s->bins[0] - 1;
        if (y > s->bins[1] - 1) y = s->bins[1] - 1;
        if (z > s->bins[2] - 1) z = s->bins[2] - 1;
        const int bin = (int)(((size_t)z * (size_t)s->bins[1] + (size_t)y) * (size_t)s->bins[0]
                              + (size_t)x);
        s->atom_bins[atom] = bin;
        bin_sizes[bin] += 1;
    }
    int running = 0;
    for (int bin = 0; bin <= num_bins; ++bin) {
        s->bin_offsets[bin] = running;
        if (bin < num_bins) running += bin_sizes[bin];
    }
    /* Fill in atom order, then insertion-sort each bin ascending: the final
     * order is ascending atom index whatever the fill order was. */
    for (int bin = 0; bin < num_bins; ++bin) bin_sizes[bin] = s->bin_offsets[bin];
    for (int atom = 0; atom < num_nodes; ++atom)
        s->bin_atoms[bin_sizes[s->atom_bins[atom]]++] = atom;
    free(bin_sizes);
    for (int bin = 0; bin < num_bins; ++bin) {
        const int begin = s->bin_offsets[bin];
        const int end = s->bin_offsets[bin + 1];
        for (int index = begin + 1; index < end; ++index) {
            const int atom = s->bin_atoms[index];
            int insertion = index;
            while (insertion > begin && s->bin_atoms[insertion - 1] > atom) {
                s->bin_atoms[insertion] = s->bin_atoms[insertion - 1];
                --insertion;
            }
            s->bin_atoms[insertion] = atom;
        }
    }
    return NB_OK;
}

/* Visits the edges of one receiver in the reference order.  With fill set,
 * writes them at ``out_offset``; returns the edge count. */
static long long nb_receiver(const nb_state* s, int receiver, int fill, long long out_offset,
                             int* sources, int* shifts, double* fractional_xyz)
{
    const int bx = s->bins[0], by = s->bins[1], bz = s->bins[2];
    const int receiver_bin = s->atom_bins[receiver];
    const int receiver_x = receiver_bin % bx;
    const int receiver_y = (receiver_bin / bx) % by;
    const int receiver_z = (int)((size_t)receiver_bin / ((size_t)bx * (size_t)by));
    long long local_edge = 0;
    for (int dz = -s->reach[2]; dz <= s->reach[2]; ++dz) {
        const int raw_z = receiver_z + dz;
        const int shift_z = floor_div(raw_z, bz);
        const int source_z = raw_z - shift_z * bz;
        for (int dy = -s->reach[1]; dy <= s->reach[1]; ++dy) {
            const int raw_y = receiver_y + dy;
            const int shift_y = floor_div(raw_y, by);
            const int source_y = raw_y - shift_y * by;
            for (int dx = -s->reach[0]; dx <= s->reach[0]; ++dx) {
                const int raw_x = receiver_x + dx;
                const int shift_x = floor_div(raw_x, bx);
                const int source_x = raw_x - shift_x * bx;
                const int source_bin = (int)(((size_t)source_z * (size_t)by + (size_t)source_y)
                                                 * (size_t)bx + (size_t)source_x);
                const int image[3] = {shift_x, shift_y, shift_z};
                for (int index = s->bin_offsets[source_bin]; index < s->bin_offsets[source_bin + 1];
                     ++index) {
                    const int source = s->bin_atoms[index];
                    if (source == receiver && shift_x == 0 && shift_y == 0 && shift_z == 0)
                        continue;
                    double distance_squared = 0.0;
                    for (int component = 0; component < 3; ++component) {
                        double displacement = s->wrapped_positions[3 * source + component]
                                              - s->wrapped_positions[3 * receiver + component];
                        for (int axis = 0; axis < 3; ++axis)
                            displacement += image[axis] * s->cell[3 * axis + component];
                        distance_squared += displacement * displacement;
                    }
                    if (distance_squared > s->cutoff_squared) continue;
                    if (fill) {
                        const long long edge = out_offset + local_edge;
                        sources[edge] = source;
                        for (int axis = 0; axis < 3; ++axis) {
                            shifts[3 * edge + axis] = image[axis] - s->wrap_shifts[3 * source + axis]
                                                      + s->wrap_shifts[3 * receiver + axis];
                            fractional_xyz[3 * edge + axis] =
                                s->wrapped_fractional[3 * source + axis]
                                - s->wrapped_fractional[3 * receiver + axis] + image[axis];
                        }
                    }
                    ++local_edge;
                }
            }
        }
    }
    return local_edge;
}

/* Counts edges per receiver.  num_neigh (N) and receiver_offsets (N+1) are
 * written; the total is returned in *num_edges. */
int oracle_neighbor_count(const double* positions, int num_nodes, const double* cell,
                          const double* inverse_cell, double cutoff, int* num_neigh,
                          int* receiver_offsets, long long* num_edges)
{
    nb_state s;
    int status = nb_prepare(&s, positions, num_nodes, cell, inverse_cell, cutoff);
    if (status != NB_OK) return status;
    long long total = 0;
    receiver_offsets[0] = 0;
    for (int receiver = 0; receiver < num_nodes; ++receiver) {
        const long long count = nb_receiver(&s, receiver, 0, 0, NULL, NULL, NULL);
        total += count;
        if (total > 2147483647LL) {
            nb_free(&s);
            nb_last_error = "neighbor graph exceeds 32-bit edge indexing";
            return NB_LENGTH_ERROR;
        }
        num_neigh[receiver] = (int)count;
        receiver_offsets[receiver + 1] = (int)total;
    }
    *num_edges = total;
    nb_free(&s);
    return NB_OK;
}

/* Fills sources (E), shifts (E x 3) and fractional_xyz (E x 3) for the edge
 * count previously returned by oracle_neighbor_count. */
int oracle_neighbor_fill(const double* positions, int num_nodes, const double* cell,
                         const double* inverse_cell, double cutoff, const int* receiver_offsets,
                         int* sources, int* shifts, double* fractional_xyz)
{
    nb_state s;
    int status = nb_prepare(&s, positions, num_nodes, cell, inverse_cell, cutoff);
    if (status != NB_OK) return status;
    for (int receiver = 0; receiver < num_nodes; ++receiver)
        nb_receiver(&s, receiver, 1, receiver_offsets[receiver], sources, shifts, fractional_xyz);
    nb_free(&s);
    return NB_OK;
}
