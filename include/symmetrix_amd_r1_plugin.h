/* R1 HIP plugin ABI, version 1: the reference's operator boundary for the
 * second-interaction edge stage (symmetrix/source/symmetrix/
 * jit_hip_plugin_abi.h:1-269).  The reference's evaluator dlopens one plugin
 * library per model contract, calls symmetrix_jit_hip_plugin_query_v1() and
 * launches r1_forward_launch (the receiver-owned tensor product,
 * jit_codegen.py:884-1016) and r1_coordinate_reverse_launch (the source-owned
 * feature adjoint and the edge-owned directed forces, jit_codegen.py:
 * 1018-1110, 1314-1424) on its own stream.  The structures below repeat the
 * reference's layouts field for field, which is what the loader binds; this
 * build ships the ahead-of-time plugin libsymmetrix_amd_r1_<contract>.so for
 * gfx950 (symmetrix-xl_amd/csrc/r1_plugin.hip).  Only the shared-plugin
 * packets are declared; the reference's module-only experimental packets
 * (tiled and projected forms) are not part of this ABI. */
#ifndef SYMMETRIX_AMD_R1_PLUGIN_H
#define SYMMETRIX_AMD_R1_PLUGIN_H

#include <stdint.h>

#define SYMMETRIX_JIT_HIP_PLUGIN_ABI_VERSION_V1 1u
#define SYMMETRIX_JIT_HIP_PLUGIN_BYTE_ORDER 0x01020304u /* little endian */
#define SYMMETRIX_JIT_HIP_PLUGIN_ABI_TAG_V1 "symmetrix.jit.hip-plugin/1"
#define SYMMETRIX_JIT_HIP_PLUGIN_QUERY_SYMBOL_V1 "symmetrix_jit_hip_plugin_query_v1"

#ifdef __cplusplus
extern "C" {
#endif

enum SymmetrixJitHipScalarKindV1 { SYMMETRIX_JIT_HIP_SCALAR_FLOAT32_V1 = 1u, SYMMETRIX_JIT_HIP_SCALAR_FLOAT64_V1 = 2u };

enum SymmetrixJitHipPluginCapabilityV1 {
    SYMMETRIX_JIT_HIP_R1_FORWARD_LAUNCH_V1 = 1u << 0,
    SYMMETRIX_JIT_HIP_R1_COORDINATE_REVERSE_LAUNCH_V1 = 1u << 1,
    SYMMETRIX_JIT_HIP_R1_FUSED_REVERSE_LAUNCH_V1 = 1u << 2
};

/* Cubic pieces c0 + c1 x + c2 x^2 + c3 x^3 (x in [0, h] from the interval's
 * knot) of `functions` radial functions per edge type (unordered active-type
 * pair), at coefficients[((edge_type intervals + interval) 4 + q) functions
 * + function]; function = path channels + channel. */
typedef struct SymmetrixJitHipRadialSplineV1 {
    uint32_t struct_size;
    uint32_t edge_types;
    uint32_t intervals;
    uint32_t functions;
    double h;
    double x0;
    const void* coefficients;
} SymmetrixJitHipRadialSplineV1;

/* Device arrays, row-major; the structure itself is read on the host.
 * Receiver-major CSR (first_neigh, num_neigh, neigh_indices, neigh_types;
 * node and neighbour types are model element indices, type_to_active maps
 * them to active-type indices), edge lengths radius [E], edge harmonics
 * harmonics_values [E][(edge_l_max + 1)^2], source features
 * neighbor_features [N][(source_l_max + 1)^2][channels]; output
 * [N][output components][channels] is overwritten.  Edges with radius >=
 * cutoff contribute nothing. */
typedef struct SymmetrixJitHipR1ForwardArgsV1 {
    uint32_t struct_size;
    uint32_t active_type_count;
    int64_t num_nodes;
    int64_t num_edges;
    const int32_t* node_types;
    const int32_t* num_neigh;
    const int32_t* first_neigh;
    const int32_t* neigh_indices;
    const int32_t* neigh_types;
    const int32_t* type_to_active;
    const double* radius;
    SymmetrixJitHipRadialSplineV1 radial;
    const void* harmonics_values;
    const void* neighbor_features;
    void* output;
    double cutoff;
} SymmetrixJitHipR1ForwardArgsV1;

/* Source-major transpose (source_offsets [N+1], source_edges, edge_receivers
 * [E]) and the output adjoint [N][output components][channels];
 * source_adjoint [N][(source_l_max + 1)^2][channels] is accumulated. */
typedef struct SymmetrixJitHipR1SourceArgsV1 {
    uint32_t struct_size;
    uint32_t active_type_count;
    int64_t num_nodes;
    int64_t num_edges;
    const int32_t* node_types;
    const int32_t* neigh_types;
    const int32_t* source_offsets;
    const int32_t* source_edges;
    const int32_t* edge_receivers;
    const int32_t* type_to_active;
    const double* radius;
    SymmetrixJitHipRadialSplineV1 radial;
    const void* harmonics_values;
    const void* output_adjoint;
    void* source_adjoint;
    double cutoff;
} SymmetrixJitHipR1SourceArgsV1;

/* Edge vectors xyz [E][3] (double, or unit vectors of coordinate_scalar_size
 * bytes when coordinates_are_unit), harmonic gradients [E][3][(edge_l_max +
 * 1)^2] (or null: formed from xyz); directed_forces [E][3] (double) has
 * -dE/dxyz subtracted, E = <output_adjoint, output>. */
typedef struct SymmetrixJitHipR1EdgeArgsV1 {
    uint32_t struct_size;
    uint32_t active_type_count;
    uint32_t coordinate_scalar_size;
    uint32_t coordinates_are_unit;
    int64_t num_nodes;
    int64_t num_edges;
    const int32_t* node_types;
    const int32_t* neigh_indices;
    const int32_t* neigh_types;
    const int32_t* edge_receivers;
    const int32_t* type_to_active;
    const void* xyz;
    const double* radius;
    SymmetrixJitHipRadialSplineV1 radial;
    const void* harmonics_values;
    const void* harmonics_gradients;
    const void* neighbor_features;
    const void* output_adjoint;
    double* directed_forces;
    double cutoff;
} SymmetrixJitHipR1EdgeArgsV1;

/* stream: the caller's hipStream_t; the last argument caps the grid
 * (persistent blocks).  Return the hipError_t of the launch; no argument
 * pointer is kept. */
typedef int32_t (*SymmetrixJitHipR1ForwardLaunchV1)(const SymmetrixJitHipR1ForwardArgsV1*, void*, int32_t);
typedef int32_t (*SymmetrixJitHipR1CoordinateReverseLaunchV1)(const SymmetrixJitHipR1SourceArgsV1*,
                                                             const SymmetrixJitHipR1EdgeArgsV1*, void*, int32_t);

typedef struct SymmetrixJitHipPluginV1 {
    uint32_t abi_version;
    uint32_t struct_size;
    uint32_t pointer_size;
    uint32_t byte_order;
    uint32_t capabilities;
    uint32_t scalar_kind;
    uint32_t scalar_size;
    uint32_t reserved;
    const char* abi_tag;
    const char* artifact_id;
    const char* contract_fingerprint;
    const char* semantic_fingerprint;
    const char* structure_fingerprint;
    int32_t channels;
    int32_t embedding;
    int32_t edge_l_max;
    int32_t source_l_max;
    const char* target_architecture;
    const char* target_features;
    int32_t native_subgroup_width;
    int32_t forward_threads_per_block;
    int32_t source_threads_per_block;
    int32_t edge_threads_per_block;
    int32_t persistent_blocks_per_compute_unit;
    SymmetrixJitHipR1ForwardLaunchV1 r1_forward_launch;
    SymmetrixJitHipR1CoordinateReverseLaunchV1 r1_coordinate_reverse_launch;
} SymmetrixJitHipPluginV1;

typedef const SymmetrixJitHipPluginV1* (*SymmetrixJitHipPluginQueryV1)(void);

/* Exported by every libsymmetrix_amd_r1_<contract>.so (no counterpart in
 * libsymmetrix_amd.so): the descriptor of that contract's plugin. */
__attribute__((visibility("default"))) const SymmetrixJitHipPluginV1* symmetrix_jit_hip_plugin_query_v1(void);

#ifdef __cplusplus
}
#endif

#endif
