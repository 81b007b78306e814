// Host/device interface of the matrix-core SOAP kernels (soap_mfma.hip).
#pragma once

#include "mdx_internal.h"

namespace mdx {

// Shape of one SOAP plan as the MFMA kernels see it.
struct MfmaDims {
    int S, n, l_max, L, H;
    int tiles;     // 16x16 contraction tiles in use
    int mode;      // 0 off, 1 inner, 2 outer
    int out_dtype; // 4 or 8
    int hpad;      // padded harmonic row: each l block rounded up to a multiple of 4
    int cpitch;    // LDS row pitch of the coefficients (hpad, or quad_coefficient_pitch)
    int clamp;     // 1 when some radial exponent argument can fall below -700
    int64_t F;
    // harmonic m-columns computed by each wavefront of a workgroup (bit m of
    // harm_mask[w]), balanced by recurrence length
    uint32_t harm_mask[16];
    // options (mdx_soap_options): S above is the graph's species; Sc the
    // coefficient species (1 for mu2); crow the LDS coefficient rows: Sc*n
    // channels, then n species-summed rows for mu1nu1, then one zero row
    int Sc;
    int compression; // 0 off, 1 mu2, 2 mu1nu1, 3 crossover
    int crow;
    int radial;      // 0 GTO, 1 polynomial
    int grid;        // polynomial radial grid points
    int weighted;    // 1 when any neighbour weight can differ from 1
    int weighting;   // 0 none, 1 poly, 2 pow, 3 exp
    int has_w0;
    double w_r0, w_c, w_d, w_m, w_w0, eta;
};

// Device tables built once per plan.
//   row_channel[t*16 + r]  radial channel l*n + k of row r of tile t, or -1
//   col_harmonic[t*16 + c] harmonic index l*l + m' of column c, or -1
//   beta_lane[(t*4 + s)*64 + lane]  A operand of beta-fold step s for a lane:
//       pi^1.5 beta[l][n'][k] pref[l][k] for row (l, n') = lane%16 and column
//       (l, k) = 4s + lane/16 of the same diagonal block, else 0 (the radial
//       prefactor is applied here, once per centre, instead of per neighbour)
//   fbase/fstride[i*W + j] feature index of channel pair (i, j), i <= j, at
//       degree l is fbase + l * fstride (layout of soap.cpp:997-1013)
struct MfmaTables {
    const int32_t* row_channel;
    const int32_t* col_harmonic;
    const double* beta_lane;
    const double* pref;
    const double* expo;
    const double* hnorm;
    const double* ps_pref;
    const int32_t* fbase;
    const int32_t* fstride;
    const double* species_w;  // species weights [S]
    const double* poly_bw;    // polynomial: w_q r_q^2 g_k(r_q), [q * n + k]
    const double* poly_grid;  // polynomial: r_q
    const int32_t* bin_atom;  // atom of each binned image (exact-self test for w0)
    const int32_t* bin_image; // image of each binned image
    const ImageDesc* images;  // image table (integer shifts)
};

// Host-side tables of a plan: block-diagonal packing of the (l, k) x (l, m)
// blocks into 16x16 tiles, the beta-fold operands and feature indices.
// beta_scaled is pi^1.5 beta with index (l*n + n')*n + k; pref is the radial
// prefactor of channel l*n + k.
struct MfmaPlanHost {
    int tiles = 0;
    std::vector<int32_t> row_channel, col_harmonic, fbase, fstride;
    std::vector<double> beta_lane;
};
MfmaPlanHost plan_mfma_tables(int S, int n, int l_max, const std::vector<double>& beta_scaled,
                              const std::vector<double>& pref);

int mfma_template_tiles(int tiles);

// 4x4-block kernel (soap_quad.hip) for the default options.  Limits: n <= 8
// (at most two radial groups of 4 channels), l_max <= kQuadLmax, at most
// kQuadMaxWaves wavefronts and kQuadG MFMA instructions per wavefront and step.
constexpr int kQuadG = 4;
// smallest radial exponent argument -a d^2 the kernel's exp accepts (its
// result must be a normal number)
constexpr double kQuadMinArgument = -700.0;
constexpr int kQuadLmax = 10;
constexpr int kQuadMaxWaves = 8;
// rows of one centre the kernel's slot codes hold (row * 16 + species in 32 bits)
constexpr int64_t kQuadMaxRows = int64_t(1) << 27;

// Constants of one lane of one wavefront of the 4x4-block kernel.
//   exp_scale  -a_lk 64/ln2 for the radial exponent a_lk of the lane's
//            A-operand row (k = 4 group + lane % 4 of its block's unit), 0 for
//            pad rows and idle blocks
//   beta_r   beta-fold A operand for the block's own accumulator:
//            pi^1.5 beta[l][n'][k] pref[l][k], n' = 4 group + lane % 4,
//            k = 4 group + lane / 16
//   beta_s   the same for the partner block's accumulator (k of the other
//            radial group; KG = 2 only)
//   ycol[g]  harmonic read by the lane for instruction g (0 where the result
//            is not stored or is scaled by 0)
//   cdst     LDS offset (within a species block of c) of the lane's fold
//            output for g = 0, + 4 g for instruction g; -1: not stored
//   cnt      instructions in which the lane's block is active
struct QuadLane {
    double exp_scale = 0.0, beta_r = 0.0, beta_s = 0.0;
    int32_t ycol[kQuadG] = {};
    int32_t cdst = -1, cnt = 0;
};

// LDS coefficient rows of the 4x4-block kernel: S*n channels, plus a zero row
// for the Gram tiles' pad channels unless S*n is a multiple of 16
inline int quad_coefficient_rows(int S, int n) { return S * n + ((S * n) % 16 != 0 ? 1 : 0); }
// LDS row pitch of the 4x4-block kernel's coefficients: odd, so that the 16
// rows of a Gram-tile operand read fall in 16 different LDS banks
inline int quad_coefficient_pitch(int hpad) { return hpad + 1; }

struct QuadPlanHost {
    int waves = 0;               // 0: the shape is outside the kernel's limits
    int kg = 0;                  // radial groups of 4 channels (1 or 2)
    int instr = 0;               // MFMA instructions per step, every wavefront (the largest unit)
    std::vector<int> units;      // column groups of each wavefront's largest unit
    std::vector<QuadLane> lanes; // [waves * 64]
};
QuadPlanHost plan_quad_tables(int n, int l_max, int hpad, const std::vector<double>& beta_scaled,
                              const std::vector<double>& pref, const std::vector<double>& expo);
size_t quad_lds_bytes(const MfmaDims& d);
void launch_quad_expand(hipStream_t stream, int waves, int kg, int instr, const PreparedBatch& pb, const DeviceGraph& g,
                        const QuadLane* lanes, const double* ps_pref, const int32_t* fbase, const int32_t* fstride,
                        const MfmaDims& d, const int64_t* item_begin, int64_t base, int64_t count, void* out,
                        int64_t pitch, double* partial);
// LDS coefficient rows of a plan: Sc*n channels, n summed rows for mu1nu1, one zero row
inline int mfma_coefficient_rows(int Sc, int n, int compression) { return Sc * n + (compression == 2 ? n : 0) + 1; }
int mfma_padded_row(int l_max);
size_t mfma_lds_bytes(const MfmaDims& d);
void launch_mfma_expand(hipStream_t stream, int template_tiles, const PreparedBatch& pb, const DeviceGraph& g,
                        const MfmaTables& tab, const MfmaDims& d, const int64_t* item_begin, int64_t base,
                        int64_t count, void* out, int64_t pitch, double* partial);
void launch_mfma_finalize(hipStream_t stream, const PreparedBatch& pb, const MfmaTables& tab, const MfmaDims& d,
                          const double* partial, const int64_t* struct_items, void* out, int64_t pitch);

} // namespace mdx
