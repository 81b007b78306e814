// Host/device interface of the register-coefficient SOAP kernel
// (soap_block.hip): GTO basis, no compression; atom-level rows (average
// "off"), with or without neighbour weights, or a row per structure of its
// centres' averaged coefficients (average "inner").
#pragma once

#include "mdx_internal.h"

namespace mdx {

// Stream kinds of the kernel: a row per centre; a row per structure (inner
// average) from a centre-by-centre stream; the same from a species-major
// stream over the structure's pairs (structures of at most 64 atoms); a row
// per centre with weighted neighbours; a row per centre of mu1nu1 features
// (each channel against the species-summed channels); inner averages of
// large structures in two launches: runs of a structure's centres leave
// their summed coefficient registers in partial rows (with or without
// neighbour weights), then a row per structure from the sum of its partial
// rows; outer averages of structures a workgroup each, every centre's power
// spectrum added into the structure's float64 row in LDS and the mean
// written once.
constexpr int kBlockRows = 0, kBlockInner = 1, kBlockInnerSmall = 2, kBlockRowsWeighted = 3, kBlockRowsSummed = 4,
              kBlockInnerRuns = 5, kBlockInnerFinal = 6, kBlockInnerRunsWeighted = 7, kBlockOuterLds = 8;
// largest row (features x 8 bytes) the outer mode accumulates in LDS
constexpr int64_t kBlockOuterLdsBytes = 48 * 1024;
constexpr int kBlockSmallAtoms = 64;

// Launch arguments (one struct, passed by value).
struct BlockArgs {
    const double* positions;    // f64[atoms * 3]
    const int64_t* pair_start;  // first pair row of each centre
    const int32_t* counts;      // rows per (centre, species)
    const uint32_t* pair_bin;   // bin of each pair row
    const double* bx;           // binned image positions
    const double* by;
    const double* bz;
    const double* lane_e1;      // [l][register][64]: -a_lk of the lane's exp row (float32 rows: -a_lk 256/ln2), 0 for pad rows
    const double* lane_beta;    // [l][fold term][64]: beta^T operand of the lane
    const int32_t* ps_offsets;  // [tile pair][value][64]: (byte offset at l = 0) << 9 | feature stride per l
    int S;                      // species
    int out_dtype;              // 4 or 8 bytes
    int64_t F;                  // features per row
    int64_t item_base, items, per_block; // centres, or structures when struct_offsets is set
    const int64_t* struct_offsets;       // null: a row per centre; else first centre of each structure
                                         // (+ end): a row per structure, its centres' average
    int small_structures;                // averages: every structure has at most 64 atoms
    // neighbour weights (soap_weight): distance function kind (0 none),
    // its parameters, w0 for the centre's own image, species weights
    int weighting;
    int has_w0;
    double w_r0, w_c, w_d, w_m, w_w0;
    const double* species_w;             // null: no weights
    const int32_t* bin_atom;             // atom of each binned image
    const int32_t* bin_image;            // image of each binned image (w0: the exact self pair)
    const int32_t* bin_type;             // species of each binned image
    const ImageDesc* images;             // image table (integer shifts)
    const double* row_w;                 // weighted modes: each pair row's weight, distance function
                                         // (or w0) times species weight (k_block_row_weights)
    int summed;                          // mu1nu1: spectrum against the species-summed coefficients
    int mu2;                             // mu2: every species' sums into the first species' slots
    // inner averages in two launches: the runs' launch writes partial_out
    // (struct_offsets = first centre of each run, + end), the final launch
    // reads partial_in (items = structures, struct_offsets = the batch's
    // atom offsets, part_items = each structure's partial rows, + end).  A
    // partial row holds every wavefront's coefficient registers, lane-major
    // (block_partial_width doubles).
    double* partial_out;
    const double* partial_in;
    const int64_t* part_items;
    // outer averages in LDS (items = structures, struct_offsets = the
    // batch's atom offsets, out_dtype 8: the plan's tables are those of
    // float64 rows): a row per structure, the mean of its centres' power
    // spectra, written with outer_lds bytes per value (4 or 8; 0: off)
    int outer_lds;
    void* out;
    int64_t pitch;              // bytes between output rows
};

// Plan tables of the kernel for one SOAP shape.  beta_scaled is
// pi^1.5 beta with index (l*n + n')*n + k, pref the radial prefactor of
// channel l*n + k, expo the radial exponent a_lk.
struct BlockPlanHost {
    int kg = 0;      // radial groups of 4 channels
    int ncr = 0;     // coefficient registers per (l, column group)
    int waves = 0;   // wavefronts per workgroup
    std::vector<double> lane_e1, lane_beta;
    std::vector<int32_t> ps_offsets; // packed feature offsets
};

// Fills out and returns true when (S, n, l_max) is one of the compiled shapes.
// compression: 0 off, 1 mu2 (one coefficient species: the shape of S
// species, the feature layout of one), 2 mu1nu1, 3 crossover (the feature
// layouts of soap.cpp:948-1013).
bool block_plan_tables(int S, int n, int l_max, int out_dtype, int compression, const std::vector<double>& beta_scaled,
                       const std::vector<double>& pref, const std::vector<double>& expo, BlockPlanHost& out);
void launch_block_expand(hipStream_t stream, int l_max, int kg, int ncr, const BlockArgs& a, int64_t count);
// doubles in one partial row of the runs' launch
int64_t block_partial_width(int l_max, int ncr);
// Each pair row's weight for the weighted modes, row_w[row] for the rows
// of centres [0, centres): the distance function of the neighbour's
// distance (w0 for the centre's own image under the zero shift) times its
// species weight (soap_weight, soap.cpp:389-420).  Uses the graph, position,
// weighting and species-weight fields of a.
void launch_block_row_weights(hipStream_t stream, const BlockArgs& a, int64_t centres, double* row_w);
// Zero the rows of the structures without atoms (structure averages; the
// expansion writes only the rows of structures it visits).
void launch_block_zero_rows(hipStream_t stream, const int64_t* struct_offsets, int64_t structures, void* out,
                            int64_t pitch, int64_t row_bytes);

} // namespace mdx
