// Kernels 2-4: per-centre SOAP expansion, power spectrum and the typed,
// coalesced feature write, plus the structure-level "inner"/"outer"
// reductions, on gfx950.
//
// Mathematics (GTO radial basis, compression off, default weighting) follows
// the reference CPU path, cpp/src/standalone/soap.cpp:
//   radial   R_lk(d^2) = pref_lk * exp(-expo_lk * d^2)           (:574-596, :893-898)
//   harmonic Y_lm      = real regular solid harmonics r^l Y_lm  (:26-370)
//   A[t][l][k][m]      = sum_{j in species t} R_lk(j) Y_lm(j)    (:902-914)
//   c[t][n][lm]        = pi^(3/2) sum_k beta[l][n][k] A[t][l][k][m] (:915-926)
//   p[(t1 n1)(t2 n2) l]= pi sqrt(8/(2l+1)) sum_m c c             (:997-1013)
// all in FP64; float32 output is the round-to-nearest cast of the FP64 value
// (the reference casts on the host, src/mdescriptor/core/result.py:64-87).
//
// Work decomposition: one 256-thread workgroup per work item.  For
// average="off" an item is one centre and the power spectrum is written
// straight to its output row; for "inner"/"outer" an item is a run of up to
// kItemCentres centres of one structure whose summed coefficients / power
// spectra go to a partial row, and a finalize kernel reduces the partial
// rows of each structure in a fixed order.
#include "mdx_internal.h"
#include "soap_mfma.h"
#include "soap_block.h"

#include <algorithm>
#include <cmath>

namespace mdx {

constexpr int kItemCentres = 32;

namespace {

struct SoapDims {
    int S, n, l_max, L, H, LN, CH;
    int mode;      // 0 off, 1 inner, 2 outer
    int out_dtype; // 4 or 8
    int acc_in_lds;
    int64_t F, C;
};

// 1/k for the harmonic recurrence denominators (l - m), k < 32
__constant__ double c_inv_int[32] = {
    0.0, 1.0, 1.0 / 2, 1.0 / 3, 1.0 / 4, 1.0 / 5, 1.0 / 6, 1.0 / 7, 1.0 / 8, 1.0 / 9, 1.0 / 10,
    1.0 / 11, 1.0 / 12, 1.0 / 13, 1.0 / 14, 1.0 / 15, 1.0 / 16, 1.0 / 17, 1.0 / 18, 1.0 / 19, 1.0 / 20,
    1.0 / 21, 1.0 / 22, 1.0 / 23, 1.0 / 24, 1.0 / 25, 1.0 / 26, 1.0 / 27, 1.0 / 28, 1.0 / 29, 1.0 / 30,
    1.0 / 31};

// Real regular solid harmonics of (x, y, z) for l <= l_max into out[l*l + ...]
// (layout of soap.cpp:60-69).  Column recurrence over m (Condon-Shortley
// seed (x + iy)^m (2m-1)!! (-1)^m), then upward in l:
//   (l-m) R_l^m = (2l-1) z R_{l-1}^m - (l+m-1) r^2 R_{l-2}^m
// the same polynomials as every branch of soap.cpp:101-370.  norm[l*L+m]
// holds N_lm (m = 0) and sqrt(2) N_lm (m > 0).
__device__ void solid_harmonics(double x, double y, double z, int l_max, int L, const double* norm,
                                double* out) {
    const double r2 = x * x + y * y + z * z;
    double re_mm = 1.0, im_mm = 0.0;
    for (int m = 0; m <= l_max; ++m) {
        if (m > 0) {
            const double f = -(2.0 * m - 1.0);
            const double nr = f * (x * re_mm - y * im_mm);
            const double ni = f * (x * im_mm + y * re_mm);
            re_mm = nr;
            im_mm = ni;
        }
        double re2 = re_mm, im2 = im_mm; // R_{l-2}
        // l = m
        {
            const int l = m;
            const double nf = norm[l * L + m];
            if (m == 0) {
                out[l * l + l] = nf * re_mm;
            } else {
                out[l * l + (l - m)] = nf * re_mm;
                out[l * l + (l + m)] = nf * im_mm;
            }
        }
        if (m == l_max) break;
        double re1 = (2.0 * m + 1.0) * z * re_mm;
        double im1 = (2.0 * m + 1.0) * z * im_mm;
        {
            const int l = m + 1;
            const double nf = norm[l * L + m];
            if (m == 0) {
                out[l * l + l] = nf * re1;
            } else {
                out[l * l + (l - m)] = nf * re1;
                out[l * l + (l + m)] = nf * im1;
            }
        }
        for (int l = m + 2; l <= l_max; ++l) {
            const double a = 2.0 * l - 1.0;
            const double b = (l + m - 1.0) * r2;
            const double inv = c_inv_int[l - m];
            const double re0 = (a * z * re1 - b * re2) * inv;
            const double im0 = (a * z * im1 - b * im2) * inv;
            re2 = re1;
            im2 = im1;
            re1 = re0;
            im1 = im0;
            const double nf = norm[l * L + m];
            if (m == 0) {
                out[l * l + l] = nf * re0;
            } else {
                out[l * l + (l - m)] = nf * re0;
                out[l * l + (l + m)] = nf * im0;
            }
        }
    }
}

__device__ inline int degree_of(int h) {
    int l = 0;
    while ((l + 1) * (l + 1) <= h) ++l;
    return l;
}

__device__ inline void store_value(void* out, int64_t pitch, int64_t row, int64_t f, double v, int dtype) {
    char* base = static_cast<char*>(out) + row * pitch;
    if (dtype == 4) {
        reinterpret_cast<float*>(base)[f] = static_cast<float>(v);
    } else {
        reinterpret_cast<double*>(base)[f] = v;
    }
}

// Power spectrum of coefficients c (LDS) for feature f.  Feature table:
// fa = (row offset of (t1, n1, l*l)) | (l << 24), fb = row offset of (t2, n2, l*l).
__device__ inline double power_feature(const double* c, const int32_t* fa, const int32_t* fb, const double* ps_pref,
                                       int64_t f) {
    const int32_t a = fa[f];
    const int l = a >> 24;
    const int oa = a & 0xffffff;
    const int ob = fb[f];
    double sum = 0.0;
    for (int m = 0; m < 2 * l + 1; ++m) sum = fma(c[oa + m], c[ob + m], sum);
    return ps_pref[l] * sum;
}

template <int NMAX, int HPT>
__global__ __launch_bounds__(kBlock) void k_soap_expand(
    const double* positions, const int64_t* pair_start, const int32_t* counts, const uint32_t* pair_bin,
    const double* bx, const double* by, const double* bz, const double* g_pref, const double* g_expo,
    const double* g_beta, const double* g_hnorm, const double* ps_pref, const int32_t* feat_a,
    const int32_t* feat_b, SoapDims d, const int64_t* item_begin, int64_t item_base, int64_t items, void* out,
    int64_t pitch, double* partial) {
    extern __shared__ double lds[];
    const int S = d.S, n = d.n, H = d.H, LN = d.LN, L = d.L, CH = d.CH;
    double* s_disp = lds;                 // CH * 3
    double* s_d2 = s_disp + CH * 3;       // CH
    double* s_y = s_d2 + CH;              // CH * H
    double* s_r = s_y + CH * H;           // CH * LN
    double* s_c = s_r + CH * LN;          // C
    double* s_beta = s_c + d.C;           // L * n * n
    double* s_pref = s_beta + L * n * n;  // LN
    double* s_expo = s_pref + LN;         // LN
    double* s_norm = s_expo + LN;         // L * L
    double* s_acc = s_norm + L * L;       // C (inner) or F (outer) when acc_in_lds
    const int tid = threadIdx.x;

    for (int i = tid; i < L * n * n; i += kBlock) s_beta[i] = g_beta[i];
    for (int i = tid; i < LN; i += kBlock) {
        s_pref[i] = g_pref[i];
        s_expo[i] = g_expo[i];
    }
    for (int i = tid; i < L * L; i += kBlock) s_norm[i] = g_hnorm[i];

    for (int64_t item = item_base + blockIdx.x; item < item_base + items; item += gridDim.x) {
        const int64_t first = item_begin ? item_begin[item] : item;
        const int64_t last = item_begin ? item_begin[item + 1] : item + 1;
        const int64_t width = d.mode == 1 ? d.C : d.F;
        double* part_row = partial != nullptr ? partial + item * width : nullptr;
        if (d.mode != 0) {
            if (d.acc_in_lds) {
                for (int64_t i = tid; i < width; i += kBlock) s_acc[i] = 0.0;
            } else {
                for (int64_t i = tid; i < width; i += kBlock) part_row[i] = 0.0;
            }
        }
        __syncthreads();
        for (int64_t centre = first; centre < last; ++centre) {
            const double cx = positions[centre * 3 + 0];
            const double cy = positions[centre * 3 + 1];
            const double cz = positions[centre * 3 + 2];
            int64_t species_begin = pair_start[centre];
            for (int t = 0; t < S; ++t) {
                const int64_t kt = counts[centre * S + t];
                double acc[HPT][NMAX];
#pragma unroll
                for (int u = 0; u < HPT; ++u) {
#pragma unroll
                    for (int k = 0; k < NMAX; ++k) acc[u][k] = 0.0;
                }
                for (int64_t j0 = 0; j0 < kt; j0 += CH) {
                    const int cnt = static_cast<int>(min<int64_t>(CH, kt - j0));
                    if (tid < cnt) {
                        const uint32_t b = pair_bin[species_begin + j0 + tid];
                        // same arithmetic as the graph kernel: image - centre, then d^2
                        const double dx = bx[b] - cx;
                        const double dy = by[b] - cy;
                        const double dz = bz[b] - cz;
                        s_disp[tid * 3 + 0] = dx;
                        s_disp[tid * 3 + 1] = dy;
                        s_disp[tid * 3 + 2] = dz;
                        s_d2[tid] = dx * dx + dy * dy + dz * dz;
                    }
                    __syncthreads();
                    if (tid < cnt) {
                        solid_harmonics(s_disp[tid * 3 + 0], s_disp[tid * 3 + 1], s_disp[tid * 3 + 2], d.l_max, L,
                                        s_norm, s_y + tid * H);
                    }
                    for (int e = tid; e < cnt * LN; e += kBlock) {
                        const int j = e / LN;
                        const int lk = e - j * LN;
                        s_r[e] = s_pref[lk] * exp(-s_expo[lk] * s_d2[j]);
                    }
                    __syncthreads();
#pragma unroll
                    for (int u = 0; u < HPT; ++u) {
                        const int h = tid + u * kBlock;
                        if (h < H) {
                            const int l = degree_of(h);
                            for (int j = 0; j < cnt; ++j) {
                                const double y = s_y[j * H + h];
                                const double* r = s_r + j * LN + l * n;
#pragma unroll
                                for (int k = 0; k < NMAX; ++k) {
                                    if (k < n) acc[u][k] = fma(r[k], y, acc[u][k]);
                                }
                            }
                        }
                    }
                    __syncthreads();
                }
                // fold beta (already scaled by pi^(3/2)) into c[t][n'][h]
#pragma unroll
                for (int u = 0; u < HPT; ++u) {
                    const int h = tid + u * kBlock;
                    if (h < H) {
                        const int l = degree_of(h);
                        for (int nn = 0; nn < n; ++nn) {
                            const double* brow = s_beta + (l * n + nn) * n;
                            double sum = 0.0;
#pragma unroll
                            for (int k = 0; k < NMAX; ++k) {
                                if (k < n) sum = fma(brow[k], acc[u][k], sum);
                            }
                            s_c[(static_cast<int64_t>(t) * n + nn) * H + h] = sum;
                        }
                    }
                }
                species_begin += kt;
            }
            __syncthreads();
            if (d.mode == 0) {
                for (int64_t f = tid; f < d.F; f += kBlock) {
                    store_value(out, pitch, centre, f, power_feature(s_c, feat_a, feat_b, ps_pref, f), d.out_dtype);
                }
            } else if (d.mode == 1) {
                if (d.acc_in_lds) {
                    for (int64_t i = tid; i < d.C; i += kBlock) s_acc[i] += s_c[i];
                } else {
                    for (int64_t i = tid; i < d.C; i += kBlock) part_row[i] += s_c[i];
                }
            } else {
                if (d.acc_in_lds) {
                    for (int64_t f = tid; f < d.F; f += kBlock) s_acc[f] += power_feature(s_c, feat_a, feat_b, ps_pref, f);
                } else {
                    for (int64_t f = tid; f < d.F; f += kBlock) part_row[f] += power_feature(s_c, feat_a, feat_b, ps_pref, f);
                }
            }
            __syncthreads();
        }
        if (d.mode != 0 && d.acc_in_lds) {
            for (int64_t i = tid; i < width; i += kBlock) part_row[i] = s_acc[i];
        }
        __syncthreads();
    }
}

// inner: mean of the structure's coefficients, then one power spectrum
// (soap.cpp:1019-1067); empty structures give zeros.
__global__ __launch_bounds__(kBlock) void k_finalize_inner(const double* partial, const int64_t* struct_items,
                                                          const int64_t* offsets, int64_t structures, SoapDims d,
                                                          const double* ps_pref, const int32_t* feat_a,
                                                          const int32_t* feat_b, void* out, int64_t pitch) {
    extern __shared__ double s_c[];
    for (int64_t s = blockIdx.x; s < structures; s += gridDim.x) {
        const int64_t natoms = offsets[s + 1] - offsets[s];
        const double inv = natoms > 0 ? 1.0 / static_cast<double>(natoms) : 0.0;
        const int64_t ib = struct_items[s], ie = struct_items[s + 1];
        for (int64_t i = threadIdx.x; i < d.C; i += kBlock) {
            double sum = 0.0;
            for (int64_t it = ib; it < ie; ++it) sum += partial[it * d.C + i];
            s_c[i] = natoms > 0 ? sum * inv : 0.0;
        }
        __syncthreads();
        for (int64_t f = threadIdx.x; f < d.F; f += kBlock) {
            store_value(out, pitch, s, f, power_feature(s_c, feat_a, feat_b, ps_pref, f), d.out_dtype);
        }
        __syncthreads();
    }
}

// outer: mean of the atoms' power spectra (soap.cpp:1068-1120); empty
// structures give zeros.  blockIdx.y splits a row's features over
// gridDim.y workgroups.
__global__ __launch_bounds__(kBlock) void k_finalize_outer(const double* partial, const int64_t* struct_items,
                                                          const int64_t* offsets, int64_t structures, SoapDims d,
                                                          void* out, int64_t pitch) {
    for (int64_t s = blockIdx.x; s < structures; s += gridDim.x) {
        const int64_t natoms = offsets[s + 1] - offsets[s];
        const double inv = natoms > 0 ? 1.0 / static_cast<double>(natoms) : 0.0;
        const int64_t ib = struct_items[s], ie = struct_items[s + 1];
        for (int64_t f = static_cast<int64_t>(blockIdx.y) * kBlock + threadIdx.x; f < d.F;
             f += static_cast<int64_t>(gridDim.y) * kBlock) {
            double sum = 0.0;
            for (int64_t it = ib; it < ie; ++it) sum += partial[it * d.F + f];
            store_value(out, pitch, s, f, natoms > 0 ? sum * inv : 0.0, d.out_dtype);
        }
    }
}

// Structure averages: the expansion leaves partial rows (width doubles),
// one per item of kItemCentres centres or one per centre.  A structure of
// thousands of atoms has hundreds of them or more, too many for the finalize
// kernels' one workgroup per structure to walk (16 structures of 4,096
// atoms: 1.1 ms), so they are first folded in parallel: split z of
// structure s sums the structure's rows [z * per_split, (z + 1) * per_split)
// in order into folded row s * splits + z (a split past the structure's rows
// is zero), and the finalize then walks the structure's splits (at most
// kFoldSplits).  The order of the sums is fixed, so the result does not
// depend on the launch.
constexpr int kFoldItems = 16;  // rows per split, at least
constexpr int kFoldSplits = 32; // splits per structure, at most
__global__ __launch_bounds__(kBlock) void k_fold_partials(const double* partial, int64_t width,
                                                          const int64_t* struct_items, int64_t col_tiles,
                                                          int splits, int64_t per_split, double* folded) {
    const int64_t s = blockIdx.x / col_tiles;
    const int64_t col = (blockIdx.x - s * col_tiles) * kBlock + threadIdx.x;
    if (col >= width) return;
    const int64_t ib = struct_items[s], ie = struct_items[s + 1];
    const int64_t a = ib + static_cast<int64_t>(blockIdx.y) * per_split;
    const int64_t b = min(a + per_split, ie);
    double sum = 0.0;
    for (int64_t it = a; it < b; ++it) sum += partial[it * width + col];
    folded[(s * splits + blockIdx.y) * width + col] = sum;
}

size_t expand_lds_bytes(const mdx_soap_plan& p, int CH, int acc_words) {
    const size_t words = static_cast<size_t>(CH) * 4 + static_cast<size_t>(CH) * p.H + static_cast<size_t>(CH) * p.LN
        + static_cast<size_t>(p.coeff_size) + static_cast<size_t>(p.L) * p.n * p.n + 2 * static_cast<size_t>(p.LN)
        + static_cast<size_t>(p.L) * p.L + static_cast<size_t>(acc_words);
    return words * sizeof(double);
}

template <int NMAX, int HPT>
void launch_expand(hipStream_t stream, dim3 grid, size_t lds, const mdx_soap_plan& p, const PreparedBatch& pb,
                   const DeviceGraph& g, const SoapDims& d, const int64_t* item_begin, int64_t base, int64_t count,
                   void* out, int64_t pitch, double* partial) {
    hipLaunchKernelGGL((k_soap_expand<NMAX, HPT>), grid, dim3(kBlock), lds, stream, pb.d_positions.as<double>(),
                       g.pair_start.as<int64_t>(), g.counts.as<int32_t>(), g.pair_bin.as<uint32_t>(),
                       g.bin_x.as<double>(), g.bin_y.as<double>(), g.bin_z.as<double>(), p.d_pref.as<double>(),
                       p.d_expo.as<double>(), p.d_beta.as<double>(), p.d_hnorm.as<double>(), p.d_ps_pref.as<double>(),
                       p.d_feat_a.as<int32_t>(), p.d_feat_b.as<int32_t>(), d, item_begin, base, count, out, pitch,
                       partial);
}

template <int NMAX>
void dispatch_hpt(int hpt, hipStream_t stream, dim3 grid, size_t lds, const mdx_soap_plan& p, const PreparedBatch& pb,
                  const DeviceGraph& g, const SoapDims& d, const int64_t* item_begin, int64_t base, int64_t count,
                  void* out, int64_t pitch, double* partial) {
    if (hpt == 1) {
        launch_expand<NMAX, 1>(stream, grid, lds, p, pb, g, d, item_begin, base, count, out, pitch, partial);
    } else {
        launch_expand<NMAX, 2>(stream, grid, lds, p, pb, g, d, item_begin, base, count, out, pitch, partial);
    }
}

} // namespace

void run_soap(hipStream_t stream, const mdx_soap_plan& p, PreparedBatch& pb, const DeviceGraph& g,
              void* out_device, int64_t pitch_bytes, DeviceBuffer& partials, const volatile int32_t* cancel,
              hipEvent_t* events, mdx_timing* timing, int64_t slice_items, const SliceHook* on_slice,
              hipStream_t weight_stream, hipEvent_t weight_ready) {
    SoapDims d{};
    d.S = p.S;
    d.n = p.n;
    d.l_max = p.l_max;
    d.L = p.L;
    d.H = p.H;
    d.LN = p.LN;
    d.mode = p.average;
    d.out_dtype = p.out_dtype;
    d.F = p.features;
    d.C = p.coeff_size;
    const int64_t rows = p.average != 0 ? pb.structures : pb.atoms;
    if (rows == 0 || d.F == 0) return;

    // the register-coefficient kernel where the plan chose it (atom-level
    // rows, with or without weights and with the compressions it takes, or
    // unweighted, uncompressed structure averages of the inner kind, which it
    // forms from the structure's centres directly) and every centre's rows
    // fit their slot codes
    // It forms a structure's inner average in one workgroup when the
    // structures are small (a wavefront of atoms) or many enough to fill the
    // device (four per compute unit); a batch of a few large structures (16
    // cells of 4,096 atoms: 16 workgroups, 50 ms) sums runs of centres into
    // partial coefficient rows instead, reduced per structure (1.1 ms).
    int64_t largest_structure = 0;
    for (size_t st = 0; st + 1 < pb.offsets.size(); ++st) {
        largest_structure = std::max(largest_structure, pb.offsets[st + 1] - pb.offsets[st]);
    }
    const bool inner_fits = largest_structure <= kBlockSmallAtoms || p.block_forced ||
                            pb.structures >= 4 * static_cast<int64_t>(device_compute_units());
    // Outer averages of the same large structures take it too: every
    // centre's row as a float64 partial row (at most 4 GiB of them), folded
    // per structure, then the mean (k_finalize_outer).  Many small
    // structures keep the 4x4-block kernel, whose partial rows sum runs of
    // centres in LDS (a row per centre would multiply the traffic by the
    // run length).
    const bool outer_fits = (!inner_fits || p.block_forced) && static_cast<double>(pb.atoms) * static_cast<double>(d.F) * 8.0 <= 4294967296.0;
    // Outer averages of small structures (or of more structures than fill
    // the device), unweighted and without mu1nu1, take it with a workgroup
    // per structure: each centre's power spectrum is added into the
    // structure's float64 row in LDS and the mean written once, with no
    // partial rows in HBM.
    const bool outer_lds = p.average == 2 && inner_fits && p.weighted == 0 && p.compression != 2 &&
                           d.F * static_cast<int64_t>(sizeof(double)) <= kBlockOuterLdsBytes;
    // (inner averages with neighbour weights only as runs of centres: the
    // per-structure modes do not weight)
    const bool block = p.block_waves > 0 &&
                       (p.average == 0 || (p.average == 2 && (outer_fits || outer_lds)) ||
                        (p.average == 1 && p.compression == 0 && (p.weighted == 0 || !inner_fits))) &&
                       g.row_bound < kQuadMaxRows;
    const bool block_inner = block && p.average == 1 && inner_fits;
    // other inner averages on that kernel: runs of a structure's centres
    // into partial rows, folded, then a launch of one workgroup per structure
    const bool block_runs = block && p.average == 1 && !inner_fits;
    const bool block_outer_lds = block && outer_lds;
    const bool block_outer = block && p.average == 2 && !outer_lds;

    // work items
    std::vector<int64_t>& item_begin_h = pb.item_begin;
    std::vector<int64_t>& struct_items_h = pb.struct_items;
    item_begin_h.clear();
    struct_items_h.clear();
    int64_t items = block_inner || block_outer_lds ? pb.structures : pb.atoms;
    if (block_outer) {
        // items are the centres, a structure's partial rows its atoms
        struct_items_h = pb.offsets;
    } else if (p.average != 0 && !block_inner && !block_outer_lds) {
        struct_items_h.resize(static_cast<size_t>(pb.structures) + 1);
        for (int64_t s = 0; s < pb.structures; ++s) {
            struct_items_h[static_cast<size_t>(s)] = static_cast<int64_t>(item_begin_h.size());
            for (int64_t a = pb.offsets[static_cast<size_t>(s)]; a < pb.offsets[static_cast<size_t>(s) + 1];
                 a += kItemCentres) {
                item_begin_h.push_back(a);
            }
        }
        struct_items_h[static_cast<size_t>(pb.structures)] = static_cast<int64_t>(item_begin_h.size());
        items = static_cast<int64_t>(item_begin_h.size());
        item_begin_h.push_back(pb.atoms);
    }
    DeviceBuffer& scratch = partials;
    int64_t* d_item_begin = nullptr;
    int64_t* d_struct_items = nullptr;
    double* d_partial = nullptr;
    // folded partial rows (see k_fold_partials): splits per structure, the
    // folded rows and their structure ranges
    int fold_splits = 0;
    int64_t fold_per_split = 0;
    size_t partial_width = 0;
    double* d_folded = nullptr;
    // weighted plans on the register-coefficient kernel: each pair row's
    // weight, computed once before the expansion (k_block_row_weights), after
    // any partial rows in the scratch buffer
    const size_t row_w_bytes =
        block && p.weighted != 0 ? ((g.pair_bin.bytes / sizeof(uint32_t)) * sizeof(double) + 255) & ~size_t(255) : 0;
    double* d_row_w = nullptr;
    int64_t* d_fold_items = nullptr;
    std::vector<int64_t>& fold_items_h = pb.fold_items;
    if (p.average != 0 && !block_inner && !block_outer_lds) {
        const size_t inner_width = p.use_mfma ? static_cast<size_t>(mfma_coefficient_rows(p.Sc, p.n, p.compression)) * static_cast<size_t>(p.hpad)
                                              : static_cast<size_t>(d.C);
        const size_t width = block_runs ? static_cast<size_t>(block_partial_width(p.l_max, p.block_ncr))
                             : p.average == 1 ? inner_width
                                              : static_cast<size_t>(d.F);
        partial_width = width;
        int64_t most_items = 0;
        for (int64_t s = 0; s < pb.structures; ++s) {
            most_items = std::max(most_items, struct_items_h[static_cast<size_t>(s) + 1] - struct_items_h[static_cast<size_t>(s)]);
        }
        if (most_items > 2 * kFoldItems) {
            fold_splits = static_cast<int>(std::min<int64_t>((most_items + kFoldItems - 1) / kFoldItems, kFoldSplits));
            fold_per_split = (most_items + fold_splits - 1) / fold_splits;
        }
        fold_items_h.clear();
        if (fold_splits > 0) {
            for (int64_t s = 0; s <= pb.structures; ++s) fold_items_h.push_back(s * fold_splits);
        }
        const size_t head = ((item_begin_h.size() + struct_items_h.size() + fold_items_h.size()) * sizeof(int64_t) + 255) &
                            ~size_t(255);
        const size_t partial_bytes = (static_cast<size_t>(items) * width * sizeof(double) + 255) & ~size_t(255);
        const size_t folded_bytes =
            (static_cast<size_t>(pb.structures) * static_cast<size_t>(fold_splits) * width * sizeof(double) + 255) &
            ~size_t(255);
        scratch.reserve(head + partial_bytes + folded_bytes + row_w_bytes);
        if (row_w_bytes > 0) {
            d_row_w = reinterpret_cast<double*>(static_cast<char*>(scratch.ptr) + head + partial_bytes + folded_bytes);
        }
        d_item_begin = scratch.as<int64_t>();
        d_struct_items = d_item_begin + item_begin_h.size();
        d_fold_items = d_struct_items + struct_items_h.size();
        d_partial = reinterpret_cast<double*>(static_cast<char*>(scratch.ptr) + head);
        if (fold_splits > 0) d_folded = reinterpret_cast<double*>(static_cast<char*>(scratch.ptr) + head + partial_bytes);
        if (!item_begin_h.empty()) {
            MDX_HIP(hipMemcpyAsync(d_item_begin, item_begin_h.data(), item_begin_h.size() * sizeof(int64_t),
                                   hipMemcpyHostToDevice, stream));
        }
        MDX_HIP(hipMemcpyAsync(d_struct_items, struct_items_h.data(), struct_items_h.size() * sizeof(int64_t),
                               hipMemcpyHostToDevice, stream));
        if (fold_splits > 0) {
            MDX_HIP(hipMemcpyAsync(d_fold_items, fold_items_h.data(), fold_items_h.size() * sizeof(int64_t),
                                   hipMemcpyHostToDevice, stream));
        }
    }
    if (row_w_bytes > 0 && d_row_w == nullptr) {
        scratch.reserve(row_w_bytes);
        d_row_w = scratch.as<double>();
    }
    // the partial rows the finalize kernels walk, folded first where
    // structures have many items
    auto fold = [&]() -> std::pair<const double*, const int64_t*> {
        if (fold_splits == 0) return {d_partial, d_struct_items};
        const int64_t col_tiles = (static_cast<int64_t>(partial_width) + kBlock - 1) / kBlock;
        hipLaunchKernelGGL(k_fold_partials, dim3(static_cast<unsigned>(col_tiles * pb.structures),
                                                 static_cast<unsigned>(fold_splits)),
                           dim3(kBlock), 0, stream, d_partial, static_cast<int64_t>(partial_width), d_struct_items,
                           col_tiles, fold_splits, fold_per_split, d_folded);
        MDX_HIP(hipGetLastError());
        return {d_folded, d_fold_items};
    };

    // launch in slices so cancellation is polled between launches (and, for
    // an atom-level run, so the caller can copy finished rows out meanwhile)
    const int64_t slice = slice_items > 0 ? slice_items : int64_t(1) << 17;
    const bool hook = on_slice != nullptr && *on_slice && p.average == 0;
    int64_t launches = 0;
    if (block || p.use_mfma) {
        // else the 4x4-block kernel where the plan chose it
        const bool quad = !block && p.quad_waves > 0 && g.row_bound < kQuadMaxRows;
        MfmaDims md{};
        md.S = p.S;
        md.n = p.n;
        md.l_max = p.l_max;
        md.L = p.L;
        md.H = p.H;
        md.tiles = p.tiles;
        md.mode = p.average;
        md.out_dtype = p.out_dtype;
        md.F = p.features;
        md.hpad = p.hpad;
        md.clamp = p.clamp;
        md.Sc = p.Sc;
        md.compression = p.compression;
        md.crow = quad ? quad_coefficient_rows(p.Sc, p.n) : mfma_coefficient_rows(p.Sc, p.n, p.compression);
        md.radial = p.radial_basis;
        md.grid = p.grid_size;
        md.weighted = p.weighted;
        md.weighting = p.weighting;
        md.has_w0 = p.has_w0;
        md.w_r0 = p.w_r0;
        md.w_c = p.w_c;
        md.w_d = p.w_d;
        md.w_m = p.w_m;
        md.w_w0 = p.w_w0;
        md.eta = p.eta;
        MfmaTables tab{};
        tab.row_channel = p.d_row_channel.as<int32_t>();
        tab.col_harmonic = p.d_col_harmonic.as<int32_t>();
        tab.beta_lane = p.d_beta_lane.as<double>();
        tab.pref = p.d_pref.as<double>();
        tab.expo = p.d_expo.as<double>();
        tab.hnorm = p.d_hnorm.as<double>();
        tab.ps_pref = p.d_ps_pref.as<double>();
        tab.fbase = p.d_fbase.as<int32_t>();
        tab.fstride = p.d_fstride.as<int32_t>();
        tab.species_w = p.d_species_w.as<double>();
        tab.poly_bw = p.d_poly_bw.as<double>();
        tab.poly_grid = p.d_poly_grid.as<double>();
        tab.bin_atom = g.bin_atom.as<int32_t>();
        tab.bin_image = g.bin_image.as<int32_t>();
        tab.images = pb.d_images.as<ImageDesc>();
        const int tt = mfma_template_tiles(p.tiles);
        BlockArgs block_args{};
        // (the weight pass counts with the graph's time: the expansion's
        // events bracket its own launches only)
        if (d_row_w != nullptr) {
            BlockArgs wa{};
            wa.positions = pb.d_positions.as<double>();
            wa.pair_start = g.pair_start.as<int64_t>();
            wa.counts = g.counts.as<int32_t>();
            wa.pair_bin = g.pair_bin.as<uint32_t>();
            wa.bx = g.bin_x.as<double>();
            wa.by = g.bin_y.as<double>();
            wa.bz = g.bin_z.as<double>();
            wa.S = p.S;
            wa.weighting = p.weighting;
            wa.has_w0 = p.has_w0;
            wa.w_r0 = p.w_r0;
            wa.w_c = p.w_c;
            wa.w_d = p.w_d;
            wa.w_m = p.w_m;
            wa.w_w0 = p.w_w0;
            wa.species_w = p.d_species_w.as<double>();
            wa.bin_atom = g.bin_atom.as<int32_t>();
            wa.bin_image = g.bin_image.as<int32_t>();
            wa.bin_type = g.bin_type.as<int32_t>();
            wa.images = pb.d_images.as<ImageDesc>();
            if (weight_stream != nullptr && weight_ready != nullptr) {
                // behind the graph on its own stream (it reads only the
                // graph, the positions and the plan)
                launch_block_row_weights(weight_stream, wa, pb.atoms, d_row_w);
                MDX_HIP(hipEventRecord(weight_ready, weight_stream));
                MDX_HIP(hipStreamWaitEvent(stream, weight_ready, 0));
            } else {
                launch_block_row_weights(stream, wa, pb.atoms, d_row_w);
            }
        }
        if (events != nullptr) MDX_HIP(hipEventRecord(events[2], stream));
        for (int64_t base = 0; base < items; base += slice) {
            if (cancel != nullptr && *cancel != 0) throw Error(MDX_CANCELLED, "descriptor computation was cancelled");
            const int64_t count = std::min(slice, items - base);
            if (block) {
                BlockArgs ba{};
                ba.positions = pb.d_positions.as<double>();
                ba.pair_start = g.pair_start.as<int64_t>();
                ba.counts = g.counts.as<int32_t>();
                ba.pair_bin = g.pair_bin.as<uint32_t>();
                ba.bx = g.bin_x.as<double>();
                ba.by = g.bin_y.as<double>();
                ba.bz = g.bin_z.as<double>();
                ba.lane_e1 = p.d_block_e1.as<double>();
                ba.lane_beta = p.d_block_beta.as<double>();
                ba.ps_offsets = p.d_block_ps.as<int32_t>();
                ba.S = p.S;
                ba.out_dtype = block_outer || block_outer_lds ? 8 : p.out_dtype;
                ba.F = p.features;
                ba.item_base = base;
                ba.items = count;
                ba.struct_offsets = block_inner || block_outer_lds ? pb.d_offsets.as<int64_t>()
                                    : block_runs                  ? d_item_begin
                                                                  : nullptr;
                ba.outer_lds = block_outer_lds ? p.out_dtype : 0;
                ba.partial_out = block_runs ? d_partial : nullptr;
                ba.small_structures = block_inner && largest_structure <= kBlockSmallAtoms ? 1 : 0;
                ba.summed = p.compression == 2 ? 1 : 0;
                ba.mu2 = p.compression == 1 ? 1 : 0;
                if (p.weighted != 0) {
                    ba.weighting = p.weighting;
                    ba.has_w0 = p.has_w0;
                    ba.w_r0 = p.w_r0;
                    ba.w_c = p.w_c;
                    ba.w_d = p.w_d;
                    ba.w_m = p.w_m;
                    ba.w_w0 = p.w_w0;
                    ba.species_w = p.d_species_w.as<double>();
                    ba.bin_atom = g.bin_atom.as<int32_t>();
                    ba.bin_image = g.bin_image.as<int32_t>();
                    ba.images = pb.d_images.as<ImageDesc>();
                    ba.row_w = d_row_w;
                }
                ba.out = block_outer ? static_cast<void*>(d_partial) : out_device;
                ba.pitch = block_outer ? static_cast<int64_t>(partial_width * sizeof(double)) : pitch_bytes;
                block_args = ba;
                launch_block_expand(stream, p.l_max, p.block_kg, p.block_ncr, ba, count);
            } else if (quad) {
                launch_quad_expand(stream, p.quad_waves, p.quad_kg, p.quad_instr, pb, g, p.d_quad_lanes.as<QuadLane>(),
                                   tab.ps_pref, tab.fbase, tab.fstride, md, d_item_begin, base, count, out_device,
                                   pitch_bytes, d_partial);
            } else {
                launch_mfma_expand(stream, tt, pb, g, tab, md, d_item_begin, base, count, out_device, pitch_bytes,
                                   d_partial);
            }
            ++launches;
            if (hook) (*on_slice)(base, count);
        }
        if (events != nullptr) MDX_HIP(hipEventRecord(events[3], stream));
        if (block_outer) {
            const auto rows_in = fold();
            // a workgroup per structure and 256 features
            const unsigned col_tiles = static_cast<unsigned>((d.F + kBlock - 1) / kBlock);
            hipLaunchKernelGGL(k_finalize_outer,
                               dim3(static_cast<unsigned>(std::min<int64_t>(pb.structures, 1 << 20)), std::min(col_tiles, 65535u)),
                               dim3(kBlock), 0, stream, rows_in.first, rows_in.second, pb.d_offsets.as<int64_t>(),
                               pb.structures, d, out_device, pitch_bytes);
            MDX_HIP(hipGetLastError());
        } else if (block_runs) {
            // the structures' rows from their folded partial rows
            const auto rows_in = fold();
            BlockArgs fa = block_args;
            fa.partial_out = nullptr;
            fa.partial_in = rows_in.first;
            fa.part_items = rows_in.second;
            fa.struct_offsets = pb.d_offsets.as<int64_t>();
            fa.item_base = 0;
            fa.items = pb.structures;
            launch_block_expand(stream, p.l_max, p.block_kg, p.block_ncr, fa, pb.structures);
        } else if (block_inner || block_outer_lds) {
            // rows of structures without atoms (the expansion visits none of them)
            bool empty = false;
            for (int64_t st = 0; st < pb.structures && !empty; ++st) {
                empty = pb.offsets[static_cast<size_t>(st) + 1] == pb.offsets[static_cast<size_t>(st)];
            }
            if (empty) {
                launch_block_zero_rows(stream, pb.d_offsets.as<int64_t>(), pb.structures, out_device, pitch_bytes,
                                       p.features * p.out_dtype);
            }
        } else if (p.average != 0) {
            const auto rows_in = fold();
            launch_mfma_finalize(stream, pb, tab, md, rows_in.first, rows_in.second, out_device, pitch_bytes);
        }
        if (events != nullptr) MDX_HIP(hipEventRecord(events[4], stream));
        if (timing != nullptr) {
            timing->expansion_launches = launches;
            timing->expansion_tiles = block ? -(1000 + p.block_waves) : quad ? -p.quad_waves : tt;
        }
        return;
    }
    const int64_t acc_words = p.average == 1 ? d.C : p.average == 2 ? d.F : 0;
    // chunk of neighbours staged per step: largest that keeps LDS within budget
    const size_t budget = 64 * 1024;
    int CH = 64;
    while (CH > 8 && expand_lds_bytes(p, CH, 0) > budget) CH /= 2;
    d.CH = CH;
    d.acc_in_lds = acc_words > 0 && expand_lds_bytes(p, CH, static_cast<int>(acc_words)) <= 96 * 1024 ? 1 : 0;
    const size_t lds = expand_lds_bytes(p, CH, d.acc_in_lds ? static_cast<int>(acc_words) : 0);
    if (lds > 160 * 1024) throw Error(MDX_INVALID_ARGUMENT, "SOAP shape exceeds the device LDS budget");

    const int hpt = p.H > kBlock ? 2 : 1;
    if (events != nullptr) MDX_HIP(hipEventRecord(events[2], stream));
    for (int64_t base = 0; base < items; base += slice) {
        if (cancel != nullptr && *cancel != 0) throw Error(MDX_CANCELLED, "descriptor computation was cancelled");
        const int64_t count = std::min(slice, items - base);
        const dim3 grid(static_cast<unsigned>(count));
        if (p.n <= 8) {
            dispatch_hpt<8>(hpt, stream, grid, lds, p, pb, g, d, d_item_begin, base, count, out_device, pitch_bytes,
                            d_partial);
        } else {
            dispatch_hpt<16>(hpt, stream, grid, lds, p, pb, g, d, d_item_begin, base, count, out_device, pitch_bytes,
                             d_partial);
        }
        MDX_HIP(hipGetLastError());
        ++launches;
        if (hook) (*on_slice)(base, count);
    }
    if (events != nullptr) MDX_HIP(hipEventRecord(events[3], stream));
    if (p.average != 0) {
        const unsigned grid = static_cast<unsigned>(std::min<int64_t>(pb.structures, 1 << 20));
        const auto rows_in = fold();
        if (p.average == 1) {
            hipLaunchKernelGGL(k_finalize_inner, dim3(grid), dim3(kBlock), static_cast<size_t>(d.C) * sizeof(double),
                               stream, rows_in.first, rows_in.second, pb.d_offsets.as<int64_t>(), pb.structures, d,
                               p.d_ps_pref.as<double>(), p.d_feat_a.as<int32_t>(), p.d_feat_b.as<int32_t>(), out_device,
                               pitch_bytes);
        } else {
            hipLaunchKernelGGL(k_finalize_outer, dim3(grid), dim3(kBlock), 0, stream, rows_in.first, rows_in.second,
                               pb.d_offsets.as<int64_t>(), pb.structures, d, out_device, pitch_bytes);
        }
        MDX_HIP(hipGetLastError());
    }
    if (events != nullptr) MDX_HIP(hipEventRecord(events[4], stream));
    if (timing != nullptr) {
        timing->expansion_launches = launches;
        timing->expansion_tiles = 0;
    }
}

} // namespace mdx
