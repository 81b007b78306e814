// Kernels 2-4 on the FP64 matrix cores of gfx950 (v_mfma_f64_16x16x4f64).
//
// One workgroup owns one centre (or one run of centres of a structure for
// the "inner"/"outer" averages), with one wavefront per contraction tile.
// Rows of kernel 1 are grouped by species; each species segment of the
// centre's list is padded to a multiple of 4 slots and the slots are walked
// in chunks of 32 that may span segments:
//
//   contraction  A[(l,k)][(l,m)] = sum_j R_lk(j) Y_lm(j)      (soap.cpp:902-914)
//     The (l,k) x (l,m) products are packed block-diagonally into 16x16
//     tiles (rows = radial channels, columns = harmonics, several l per
//     tile); each MFMA adds 4 neighbours (K = 4).  Wavefront t owns tile t:
//     a lane feeds the radial value of its tile row, so every exp(-a d^2)
//     is evaluated once, in the lane that consumes it.  The harmonics of a
//     chunk of 32 neighbours are computed two lanes per neighbour (cos/sin
//     parts), the m-columns split across the wavefronts, and staged in LDS.
//   beta fold    c = blockdiag(pi^1.5 beta_l) A               (soap.cpp:915-926)
//     The accumulator layout of the MFMA (lane L, register r holds row
//     L/16 + 4r, column L%16) is exactly the B-operand layout of step r, so
//     the fold is 4 more MFMAs per tile with no data movement.
//   power spectrum p_l = c_l c_l^T per l on 16x16 Gram tiles   (soap.cpp:997-1013)
//     reading c from LDS, scaled by pi sqrt(8/(2l+1)) and written in the
//     output dtype straight to the feature row.
//
// MFMA lane layouts (measured on gfx950): A operand lane L = A[L%16][L/16],
// B operand lane L = B[L/16][L%16], result lane L register r =
// D[L/16 + 4r][L%16].
#include "soap_device.h"

#include <algorithm>
#include <array>
#include <cmath>

namespace mdx {

static_assert(kHarmonicLmax == kMaxLmax, "harmonic table must cover every supported l_max");

namespace {

// exp(x) for the radial Gaussians, x = -a d^2 <= 0, by the table-driven
// method of P. T. P. Tang (ACM TOMS 15(2), 1989): x = (64k + j) ln2/64 + r
// with |r| <= ln2/128, exp(x) = 2^k 2^(j/64) e^r, e^r - 1 by its degree-5
// Taylor polynomial (truncation below 4e-17 relative; 2 ulp worst case
// measured against libm over [-700, 0]).  tab64[j] = 2^(j/64).  Arguments
// below -700 are clamped there (e^-700 ~ 1e-304, below every tolerance),
// which keeps 2^k a normal number.
__device__ inline double exp_neg(double x, const double* tab64) {
    constexpr double kInvLn2x64 = 92.332482616893658071035179584121;  // 64 / ln 2
    constexpr double kLn2by64Hi = 0.010830417275428772;               // ln2/64 with 32 trailing zero bits
    constexpr double kLn2by64Lo = 7.420820373486988e-09;              // ln2/64 - kLn2by64Hi
    constexpr double kShifter = 6755399441055744.0;                  // 1.5 * 2^52
    x = fmax(x, -700.0);
    const double s = fma(x, kInvLn2x64, kShifter);
    const double kf = s - kShifter;
    double r = fma(kf, -kLn2by64Hi, x);
    r = fma(kf, -kLn2by64Lo, r);
    const int ki = __double2loint(s);
    double q = fma(r, 1.0 / 120.0, 1.0 / 24.0);
    q = fma(q, r, 1.0 / 6.0);
    q = fma(q, r, 0.5);
    q = fma(q, r, 1.0);
    const double em1 = r * q;  // e^r - 1
    const double t = tab64[ki & 63];
    return ldexp(fma(t, em1, t), ki >> 6);
}

// Weight of one neighbour (soap_weight, soap.cpp:389-420): the distance
// function, w0 for the centre's own image, times the species weight.
__device__ inline double neighbour_weight(const MfmaDims& d, double distance, bool exact_self, double species_w) {
    double value = weight_function(d.weighting, d.w_r0, d.w_c, d.w_d, d.w_m, distance);
    if (exact_self && d.has_w0) value = d.w_w0;
    return value * species_w;
}

// Radial functions of the polynomial basis for the chunk's slots:
//   G[slot][l*n + k] = sum_q K_l(q; r_slot) w_q r_q^2 g_k(r_q),
// K_l the Gaussian-smeared radial kernel of polynomial_flir
// (soap.cpp:450-492) with its l = 0 special case at r <= 1e-14.  Four grid
// points at a time: one thread per (slot, point) evaluates K_0..K_lmax into
// s_f, then each (l, 16-slot tile) unit -- one wavefront's -- adds its
// 16 slots x 4 points x n product, computed on the matrix cores, into s_g.
// All threads take part (barriers inside).
__device__ void polynomial_radial(const double* s_r, double* s_f, double* s_g, const MfmaTables& tab,
                                  const MfmaDims& d, int tid, int wave, int threads, int waves) {
    const int lane = tid % kWaveThreads;
    const int L = d.L, n = d.n, Q = d.grid;
    const int GP = L * n + 1;
    constexpr int kF = kNb * 4;  // entries of one l in s_f
    for (int i = tid; i < kNb * GP; i += threads) s_g[i] = 0.0;
    for (int q0 = 0; q0 < Q; q0 += 4) {
        // (a workgroup of one wavefront takes two items per thread)
        for (int item = tid; item < kF; item += threads) {
            const int slot = item / 4, qq = item - slot * 4, q = q0 + qq;
            double* f = s_f + slot * 4 + qq;
            if (q < Q) {
                const double radius = s_r[slot];
                const double radial = tab.poly_grid[q];
                const double eta = d.eta;
                if (radius <= 1e-14) {
                    const double radial2 = radial * radial;
                    f[0] = exp(-eta * radial2);
                    for (int l = 1; l < L; ++l) f[l * kF] = 0.0;
                } else {
                    const double prefactor = 0.25 / (eta * radius * radial);
                    const double minus = exp(-eta * (radial - radius) * (radial - radius));
                    const double plus = exp(-eta * (radial + radius) * (radial + radius));
                    double before = prefactor * (minus - plus);
                    f[0] = before;
                    if (L > 1) {
                        double last = prefactor * (minus + plus - 2.0 * before);
                        f[kF] = last;
                        for (int l = 2; l < L; ++l) {
                            const double value = before - prefactor * (4.0 * l - 2.0) * last;
                            const double kept = value > 0.0 ? value : 0.0;
                            f[l * kF] = kept;
                            before = last;
                            last = kept;
                        }
                    }
                }
            } else {
                for (int l = 0; l < L; ++l) f[l * kF] = 0.0;
            }
        }
        __syncthreads();
        for (int u = wave; u < 2 * L; u += waves) {
            const int l = u >> 1, tile = u & 1;
            const double a = s_f[l * kF + (16 * tile + lane % 16) * 4 + lane / 16];
            const int q = q0 + lane / 16;
            const double b = q < Q && lane % 16 < n ? tab.poly_bw[q * n + lane % 16] : 0.0;
            const d4 g = mfma(a, b, d4{0.0, 0.0, 0.0, 0.0});
            if (lane % 16 < n) {
#pragma unroll
                for (int r = 0; r < 4; ++r) s_g[(16 * tile + lane / 16 + 4 * r) * GP + l * n + lane % 16] += g[r];
            }
        }
        __syncthreads();
    }
}

// The same radial functions with the sums over the grid in registers: up
// to kPolyDegrees degrees (L) and kPolyGroups radial groups, the common
// case.  A wavefront takes one half
// of the chunk's slots and one of P parts of the grid, four points at a
// time.  Lane L evaluates K_0..K_{L-1} for slot L % 16 of its half at grid
// point L / 16 of the four, which is the A operand of v_mfma_f64_4x4x4f64
// (block b = (L / 4) % 4 holds slots 4b..4b+3: A_b lane L = A_b[slot
// L % 4][point L / 16]); the B operand is the quadrature-weighted basis of
// radial group g (B lane L = w_q r_q^2 g_{4g + L % 4}(r_q) at point L / 16,
// the same for every block), so one MFMA per degree and radial group
// accumulates 4 slots x 4 channels per block with no padded channels, and
// no barrier sits inside the grid loop.  Result lane L holds slot
// 4b + L / 16, channel 4g + L % 4.  The parts' results go to s_g in part
// order (part 0 writes, the others add, a barrier between), so the sums do
// not depend on the schedule.
constexpr int kPolyDegrees = 8;
constexpr int kPolyGroups = 2; // radial groups of 4 channels (n <= 8)
__device__ __forceinline__ double mfma4(double a, double b, double c) {
    return __builtin_amdgcn_mfma_f64_4x4x4f64(a, b, c, 0, 0, 0);
}
__device__ void polynomial_radial_regs(const double* s_r, double* s_g, const double* s_tab, const MfmaTables& tab,
                                       const MfmaDims& d, int tid, int wave, int threads, int waves) {
    const int lane = tid % kWaveThreads;
    const int L = d.L, n = d.n, Q = d.grid;
    const int KG = (n + 3) / 4;
    const int GP = L * n + 1;
    const int parts = waves >= 2 ? waves / 2 : 1;
    const int blocks = (Q + 3) / 4;                       // grid blocks of 4 points
    const int per_part = (blocks + parts - 1) / parts;
    const int units = waves >= 2 ? 2 * parts : 1;
    const double eta = d.eta;
    // the pad entry of every slot's row stays zero
    for (int i = tid; i < kNb; i += threads) s_g[i * GP + GP - 1] = 0.0;
    for (int u0 = 0; u0 < (waves >= 2 ? 1 : 2); ++u0) {
        // one wavefront: both halves in turn; else unit = wavefront
        const int unit = waves >= 2 ? wave : u0;
        const bool active = unit < units || waves < 2;
        const int half = waves >= 2 ? unit % 2 : u0;
        const int part = waves >= 2 ? unit / 2 : 0;
        double acc[kPolyDegrees][kPolyGroups];
#pragma unroll
        for (int l = 0; l < kPolyDegrees; ++l) {
#pragma unroll
            for (int g = 0; g < kPolyGroups; ++g) acc[l][g] = 0.0;
        }
        if (active) {
            const double radius = s_r[16 * half + lane % 16];
            const int b0 = part * per_part, b1 = min(blocks, b0 + per_part);
            // two grid blocks per iteration: their table loads, exps and
            // degree recurrences are independent, so their latencies overlap
            for (int blk0 = b0; blk0 < b1; blk0 += 2) {
                double a_before[2], a_last[2], a_pref[2], bb[2][kPolyGroups];
                bool a_centre[2];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int blk = blk0 + u;
                    const int q = 4 * blk + lane / 16;
                    const bool on_grid = blk < b1 && q < Q;
                    const double radial = on_grid ? tab.poly_grid[q] : 1.0;
#pragma unroll
                    for (int g = 0; g < kPolyGroups; ++g) {
                        const int k = 4 * g + lane % 4;
                        bb[u][g] = g < KG && on_grid && k < n ? tab.poly_bw[q * n + k] : 0.0;
                    }
                    // K_l (soap.cpp:450-492): the l = 0 special case at r <= 1e-14
                    double before, last;
                    const bool at_centre = radius <= 1e-14;
                    double prefactor = 0.0;
                    if (at_centre) {
                        before = exp_neg(-eta * (radial * radial), s_tab);
                        last = 0.0;
                    } else {
                        prefactor = 0.25 / (eta * radius * radial);
                        const double minus = exp_neg(-eta * (radial - radius) * (radial - radius), s_tab);
                        const double plus = exp_neg(-eta * (radial + radius) * (radial + radius), s_tab);
                        before = prefactor * (minus - plus);
                        last = prefactor * (minus + plus - 2.0 * before);
                    }
                    if (!on_grid) {
                        before = 0.0;
                        last = 0.0;
                    }
                    a_before[u] = before;
                    a_last[u] = last;
                    a_pref[u] = prefactor;
                    a_centre[u] = at_centre;
                }
#pragma unroll
                for (int u = 0; u < 2; ++u) {
#pragma unroll
                    for (int g = 0; g < kPolyGroups; ++g) acc[0][g] = mfma4(a_before[u], bb[u][g], acc[0][g]);
                }
#pragma unroll
                for (int l = 1; l < kPolyDegrees; ++l) {
                    // every degree and radial group, without a branch: the
                    // sums of degrees past L are never stored, and groups
                    // past KG meet a zero basis
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        double value = a_last[u];
                        if (l >= 2) {
                            const double next = a_before[u] - a_pref[u] * (4.0 * l - 2.0) * a_last[u];
                            value = a_centre[u] ? 0.0 : (next > 0.0 ? next : 0.0);
                            a_before[u] = a_last[u];
                            a_last[u] = value;
                        }
#pragma unroll
                        for (int g = 0; g < kPolyGroups; ++g) acc[l][g] = mfma4(value, bb[u][g], acc[l][g]);
                    }
                }
            }
        }
        // the parts' sums, in part order
        const int slot = 16 * half + 4 * ((lane / 4) % 4) + lane / 16;
        for (int p = 0; p < parts; ++p) {
            if (active && part == p) {
#pragma unroll
                for (int l = 0; l < kPolyDegrees; ++l) {
#pragma unroll
                    for (int g = 0; g < kPolyGroups; ++g) {
                        const int k = 4 * g + lane % 4;
                        if (l < L && g < KG && k < n) {
                            double& v = s_g[slot * GP + l * n + k];
                            v = p == 0 ? acc[l][g] : v + acc[l][g];
                        }
                    }
                }
            }
            __syncthreads();
        }
    }
}

// kGeneral adds neighbour weights (kPoly: and the polynomial basis, whose
// sums over the grid hold registers of their own); without them the
// kernel keeps at least 4 wavefronts per SIMD (a 128-VGPR budget the
// compiler must fit), with them 2.
template <int T, bool kGeneral, bool kPoly>
__global__ __launch_bounds__(T * kWaveThreads, kGeneral ? 2 : 4) void k_soap_mfma(
    const double* __restrict__ positions, const int64_t* __restrict__ pair_start, const int32_t* __restrict__ counts,
    const uint32_t* __restrict__ pair_bin, const double* __restrict__ bx, const double* __restrict__ by,
    const double* __restrict__ bz, const MfmaTables tab, const double* __restrict__ ps_pref, MfmaDims d,
    const int64_t* __restrict__ item_begin, int64_t item_base,
    int64_t items, int64_t per_block, void* out, int64_t pitch, double* partial) {
    // ps_pref is a separate read-only, unaliased argument so that its
    // wave-uniform reads compile to scalar loads
    extern __shared__ double lds[];
    const int tid = threadIdx.x;
    const int lane = tid % kWaveThreads;
    // the tile this wavefront contracts (wave-uniform: keeps tile constants and
    // branches on it in scalar registers)
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWaveThreads);
    constexpr int kThreads = T * kWaveThreads;
    const int H = d.H, L = d.L, S = d.S, n = d.n;
    // Y row stride, odd so that the 32 slots of one harmonic store hit distinct
    // bank pairs; entry H stays zero
    const int HP = (H + 1) | 1;
    const int hp = d.hpad;                // padded c row
    const int cw = d.crow * hp;           // c words, including the zero row
    const int GP = L * n + 1;             // polynomial radial row; entry L*n stays zero
    double* s_y = lds;                    // kNb * HP
    double* s_d2 = s_y + kNb * HP;        // kNb: d^2 (GTO) or distance (polynomial) of the chunk's slots
    double* s_tab = s_d2 + kNb;           // 64: 2^(j/64) for exp_neg
    double* s_c = s_tab + 64;             // cw (coefficients of the current centre, padded)
    double* s_csum = s_c + cw;            // cw (inner average only)
    double* s_g = s_csum + (d.mode == 1 ? cw : 0);     // polynomial: kNb * GP radial functions
    double* s_f = s_g + (d.radial == 1 ? kNb * GP : 0); // polynomial: L * kNb * 4 radial kernels
    int* s_loff = reinterpret_cast<int*>(s_f + (d.radial == 1 ? L * kNb * 4 : 0)); // L + 1
    int* s_seg = s_loff + (L + 1);        // S + 1: first row of each species segment of the centre
    int* s_pseg = s_seg + (S + 1);        // S + 1: first slot of each segment (padded to 4)
    int* s_step = s_pseg + (S + 1);       // 1: species of the chunk's MFMA steps, 4 bits each

    if (tid < 64) s_tab[tid] = exp2(static_cast<double>(tid) / 64.0);
    for (int i = tid; i < kNb * HP; i += kThreads) s_y[i] = 0.0;
    for (int i = tid; i < cw; i += kThreads) s_c[i] = 0.0;
    if (tid == 0) {
        int off = 0;
        for (int l = 0; l <= L; ++l) {
            s_loff[l] = off;
            off += 4 * ((2 * l + 4) / 4);
        }
    }
    __syncthreads();
    // per-lane constants of this wavefront's tile: radial exponent of row
    // lane%16 (zero for pad rows, whose sums the fold multiplies by zero), Y
    // column of lane%16 (the zero entry H for pad columns), the beta-fold
    // operands (which carry the radial prefactors) and the destination of
    // result row lane/16 + 4r (or -1 off the diagonal)
    const bool has_tile = wave < d.tiles;
    int ycol = H, gcol = GP - 1, dst[4] = {-1, -1, -1, -1};
    double expo = 0.0, bfold[4] = {0.0, 0.0, 0.0, 0.0};
    if (has_tile) {
        const int rc = tab.row_channel[wave * 16 + lane % 16];
        const int ch = tab.col_harmonic[wave * 16 + lane % 16];
        ycol = ch >= 0 ? ch : H;
        gcol = rc >= 0 ? rc : GP - 1;
        expo = rc >= 0 ? tab.expo[rc] : 0.0;
        const int lh = ch >= 0 ? degree_of_harmonic(ch) : -1;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int och = tab.row_channel[wave * 16 + lane / 16 + 4 * r];
            const bool diag = och >= 0 && ch >= 0 && och / n == lh;
            dst[r] = diag ? (och % n) * hp + s_loff[lh] + (ch - lh * lh) : -1;
            bfold[r] = tab.beta_lane[(wave * 4 + r) * kWaveThreads + lane];
        }
    }
    const uint32_t hmask = d.harm_mask[wave];

    const int64_t item_first = item_base + static_cast<int64_t>(blockIdx.x) * per_block;
    const int64_t item_last = min(item_first + per_block, item_base + items);
    // centres of this workgroup: [first of item_first, end of item_last - 1)
    const int64_t range_end = item_first >= item_last ? 0 : item_begin ? item_begin[item_last] : item_last;
    // The per-centre metadata (species counts, first row, position) of the
    // next centre is loaded one centre ahead into registers with vector loads:
    // lane q < S holds count q, lanes 0-2 the position bits, lane 3 the first row.
    int pre_count = 0;
    int64_t pre_bits = 0;
    auto prefetch_centre = [&](int64_t c) {
        if (c < range_end) {
            if (lane < S) pre_count = counts[c * S + lane];
            if (lane < 3) {
                pre_bits = __double_as_longlong(positions[c * 3 + lane]);
            } else if (lane == 3) {
                pre_bits = pair_start[c];
            }
        }
    };
    if (item_first < item_last) prefetch_centre(item_begin ? item_begin[item_first] : item_first);
    for (int64_t item = item_first; item < item_last; ++item) {
        const int64_t first = item_begin ? item_begin[item] : item;
        const int64_t last = item_begin ? item_begin[item + 1] : item + 1;
        double* part_row = partial != nullptr ? partial + item * (d.mode == 1 ? static_cast<int64_t>(cw) : d.F) : nullptr;
        if (d.mode == 1) {
            for (int i = tid; i < cw; i += kThreads) s_csum[i] = 0.0;
        }
        for (int64_t centre = first; centre < last; ++centre) {
            // scalar copies (readlane): these stay live across the whole centre
            const double cx = __longlong_as_double(lane_value(pre_bits, 0));
            const double cy = __longlong_as_double(lane_value(pre_bits, 1));
            const double cz = __longlong_as_double(lane_value(pre_bits, 2));
            const int64_t centre_pairs = lane_value(pre_bits, 3);
            // species segments of this centre's rows (kernel 1 groups them by
            // species) and their slots: each segment is padded to a multiple of
            // 4 slots, so one MFMA step (4 slots) never mixes species while a
            // chunk of kNb slots may span several segments.  Exclusive prefix
            // sums over lanes q < S.
            {
                int rows = lane < S ? pre_count : 0;
                int pad = (rows + 3) & ~3;
#pragma unroll
                for (int off = 1; off < kMaxSpecies; off *= 2) {
                    const int r_up = __shfl_up(rows, off, kMaxSpecies);
                    const int p_up = __shfl_up(pad, off, kMaxSpecies);
                    if ((lane % kMaxSpecies) >= off) {
                        rows += r_up;
                        pad += p_up;
                    }
                }
                if (wave == 0 && lane < S) {
                    // inclusive sums: entry q + 1
                    s_seg[lane + 1] = rows;
                    s_pseg[lane + 1] = pad;
                    if (lane == 0) {
                        s_seg[0] = 0;
                        s_pseg[0] = 0;
                    }
                }
            }
            __syncthreads();
            // an empty species leaves its coefficients at zero (mu2: one block
            // for every species, empty only without neighbours)
            for (int q = 0; q < d.Sc; ++q) {
                const bool empty = d.Sc == S ? s_seg[q + 1] == s_seg[q] : s_seg[S] == 0;
                if (empty) {
                    double* cdst = s_c + q * n * hp;
                    for (int i = tid; i < n * hp; i += kThreads) cdst[i] = 0.0;
                }
            }
            const int slots = s_pseg[S];
            // row of slot p (-1 for a pad slot or p >= slots) and its species;
            // the species count runs over wave-uniform bounds (no divergence)
            auto slot_row = [&](int p, int& q) -> int {
                q = 0;
                for (int t = 1; t < S; ++t) q += p >= s_pseg[t] ? 1 : 0;
                const int off = p - s_pseg[q];
                return off < s_seg[q + 1] - s_seg[q] ? s_seg[q] + off : -1;
            };
            // prefetch: lane pair jj = lane/2 holds the image position of slot jj
            // of the next chunk (stale, finite values in pad slots)
            double px = 0.0, py = 0.0, pz = 0.0;
            int prow, pq;
            bool pself = false;
            // exact self image (NeighborView::exact_self, neighbor.cpp:683-689):
            // the centre's own atom under the zero shift; only w0 needs it
            auto exact_self = [&](uint32_t b) {
                if (tab.bin_atom[b] != static_cast<int32_t>(centre)) return false;
                const ImageDesc& image = tab.images[tab.bin_image[b]];
                return image.n[0] == 0 && image.n[1] == 0 && image.n[2] == 0;
            };
            {
                prow = slot_row(lane / 2, pq);
                if (prow >= 0) {
                    const uint32_t b = pair_bin[centre_pairs + prow];
                    px = bx[b];
                    py = by[b];
                    pz = bz[b];
                    if (kGeneral && d.has_w0) pself = exact_self(b);
                }
            }
            // the accumulator holds the partial contraction of species `cur`; it
            // is folded into s_c when the species changes and at the end
            int cur = -1;
            d4 acc = {0.0, 0.0, 0.0, 0.0};
            auto fold = [&](int q) {
                // c = Bbeta x A; step r uses accumulator register r as B
                double* cdst = s_c + q * n * hp;
                d4 c = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
                for (int r = 0; r < 4; ++r) c = mfma(bfold[r], acc[r], c);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (dst[r] >= 0) cdst[dst[r]] = c[r];
                }
            };
            for (int j0 = 0; j0 < slots; j0 += kNb) {
                {
                    // two lanes per slot (cos / sin parts), this wavefront's
                    // m-columns.  Every lane runs the recurrence so that control flow
                    // and coefficient loads stay wave-uniform; pad slots (and slots
                    // past the end) get all-zero harmonics, so whatever finite radial
                    // value meets them adds nothing
                    const int jj = lane / 2;
                    const int comp = lane % 2;
                    // same arithmetic as kernel 1: image - centre, then d^2
                    const double dx = px - cx;
                    const double dy = py - cy;
                    const double dz = pz - cz;
                    const double d2 = dx * dx + dy * dy + dz * dz;
                    // seed scale: 0 for pad slots, else the neighbour's weight
                    double scale = prow >= 0 ? 1.0 : 0.0;
                    if (kGeneral && d.weighted && prow >= 0) {
                        scale = neighbour_weight(d, sqrt(d2), pself, tab.species_w[pq]);
                    }
                    double hx = dx, hy = dy, hz = dz, slot_value = d2;
                    if (kPoly) {
                        // polynomial: harmonics of the direction, times 4 pi w (soap.cpp:833-836);
                        // the radial functions need the distance
                        const double radius = sqrt(d2);
                        const double inverse = radius <= 1e-14 ? 0.0 : 1.0 / radius;
                        hx = dx * inverse;
                        hy = dy * inverse;
                        hz = dz * inverse;
                        scale *= 4.0 * kPi;
                        slot_value = radius;
                    }
                    if (wave == 0) {
                        if (comp == 0) s_d2[jj] = slot_value;
                        // coefficient species of the 8 MFMA steps, 4 bits each, from the
                        // lanes holding slots 0, 4, .., 28 (lanes 0, 8, .., 56); mu2
                        // sums every species into block 0
                        const int qc = d.Sc == S ? pq : 0;
                        uint32_t bits = lane % 8 == 0 ? static_cast<uint32_t>(qc) << (4 * (lane / 8)) : 0u;
                        bits |= __shfl_xor(bits, 8);
                        bits |= __shfl_xor(bits, 16);
                        bits |= __shfl_xor(bits, 32);
                        if (lane == 0) s_step[0] = static_cast<int>(bits);
                    }
                    // l_max, the column mask and an offset of zero into the table are
                    // re-read from opaque scalar registers every chunk, so that the
                    // compiler keeps the coefficient loads and the branches on them
                    // inside the loop instead of holding their results in (spilled)
                    // scalar registers across it
                    int lm = d.l_max, zero = 0;
                    uint32_t mk = hmask;
                    asm volatile("" : "+s"(lm), "+s"(mk), "+s"(zero));
                    // likewise the lane's component, so that the per-column LDS
                    // addresses derived from it are not held across the loop
                    int part = comp;
                    asm volatile("" : "+v"(part));
                    harmonics_q(hx, hy, hz, scale, lm, mk, part, &kHarmonic + zero, s_y + jj * HP);
                }
                __syncthreads();
                if constexpr (kPoly) {
                    if (L <= kPolyDegrees && n <= 4 * kPolyGroups) {
                        polynomial_radial_regs(s_d2, s_g, s_tab, tab, d, tid, wave, kThreads, T);
                    } else {
                        polynomial_radial(s_d2, s_f, s_g, tab, d, tid, wave, kThreads, T);
                    }
                }
                {
                    // issue the loads of the next chunk now
                    prow = slot_row(j0 + kNb + lane / 2, pq);
                    if (prow >= 0) {
                        const uint32_t b = pair_bin[centre_pairs + prow];
                        px = bx[b];
                        py = by[b];
                        pz = bz[b];
                        if (kGeneral && d.has_w0) pself = exact_self(b);
                    }
                }
                if (has_tile) {
                    // per half chunk: operands of 4 steps first (independent LDS
                    // reads and exps the compiler can overlap), then their MFMAs
                    const uint32_t species = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(s_step[0]));
                    const int nst = min(kNb / 4, (slots - j0) / 4);
#pragma unroll
                    for (int h = 0; h < kNb / 4; h += 4) {
                        double av[4], yv[4];
#pragma unroll
                        for (int s = 0; s < 4; ++s) {
                            const int jj = 4 * (h + s) + lane / 16;
                            av[s] = !kPoly ? exp_neg(-expo * s_d2[jj], s_tab) : s_g[jj * GP + gcol];
                            yv[s] = s_y[jj * HP + ycol];
                        }
#pragma unroll
                        for (int s = 0; s < 4; ++s) {
                            if (h + s < nst) {
                                const int q = static_cast<int>((species >> (4 * (h + s))) & 15u);
                                if (q != cur) {
                                    if (cur >= 0) fold(cur);
                                    cur = q;
                                    acc = d4{0.0, 0.0, 0.0, 0.0};
                                }
                                acc = mfma(av[s], yv[s], acc);
                            }
                        }
                    }
                }
                __syncthreads();
            }
            if (has_tile && cur >= 0) fold(cur);
            // the next centre's metadata arrives while this one's power spectrum runs
            prefetch_centre(centre + 1);
            __syncthreads();
            if (d.compression == 2 && d.mode != 1) {
                species_sums(s_c, d, tid, kThreads);
                __syncthreads();
            }
            if (d.mode == 0) {
                power_spectrum_tiles(s_c, s_loff, d, ps_pref, 0, out, pitch, centre, nullptr, wave, T);
            } else if (d.mode == 1) {
                for (int i = tid; i < cw; i += kThreads) s_csum[i] += s_c[i];
            } else {
                power_spectrum_tiles(s_c, s_loff, d, ps_pref, centre == first ? 3 : 2, out, pitch, centre, part_row,
                                     wave, T);
            }
            __syncthreads();
        }
        if (d.mode == 1) {
            for (int i = tid; i < cw; i += kThreads) part_row[i] = s_csum[i];
        }
        __syncthreads();
    }
}

// inner average: mean coefficients of each structure, then one power spectrum
__global__ __launch_bounds__(kWaveThreads) void k_mfma_finalize_inner(const double* partial, const int64_t* struct_items,
                                                                     const int64_t* offsets, int64_t structures,
                                                                     const MfmaTables tab, MfmaDims d, void* out,
                                                                     int64_t pitch) {
    extern __shared__ double lds[];
    const int cw = d.crow * d.hpad;
    double* s_c = lds;
    int* s_loff = reinterpret_cast<int*>(s_c + cw);
    if (threadIdx.x == 0) {
        int off = 0;
        for (int l = 0; l <= d.L; ++l) {
            s_loff[l] = off;
            off += 4 * ((2 * l + 4) / 4);
        }
    }
    for (int64_t s = blockIdx.x; s < structures; s += gridDim.x) {
        const int64_t natoms = offsets[s + 1] - offsets[s];
        const double inv = natoms > 0 ? 1.0 / static_cast<double>(natoms) : 0.0;
        const int64_t ib = struct_items[s], ie = struct_items[s + 1];
        for (int i = threadIdx.x; i < cw; i += kWaveThreads) {
            double sum = 0.0;
            for (int64_t it = ib; it < ie; ++it) sum += partial[it * cw + i];
            s_c[i] = natoms > 0 ? sum * inv : 0.0;
        }
        __syncthreads();
        if (d.compression == 2) {
            species_sums(s_c, d, threadIdx.x, kWaveThreads);
            __syncthreads();
        }
        power_spectrum_tiles(s_c, s_loff, d, tab.ps_pref, 0, out, pitch, s, nullptr, 0, 1);
        __syncthreads();
    }
}

__global__ void k_mfma_finalize_outer(const double* partial, const int64_t* struct_items, const int64_t* offsets,
                                      int64_t structures, MfmaDims d, void* out, int64_t pitch) {
    for (int64_t s = blockIdx.x; s < structures; s += gridDim.x) {
        const int64_t natoms = offsets[s + 1] - offsets[s];
        const double inv = natoms > 0 ? 1.0 / static_cast<double>(natoms) : 0.0;
        const int64_t ib = struct_items[s], ie = struct_items[s + 1];
        for (int64_t f = threadIdx.x; f < d.F; f += blockDim.x) {
            double sum = 0.0;
            for (int64_t it = ib; it < ie; ++it) sum += partial[it * d.F + f];
            store_out(out, pitch, s, f, natoms > 0 ? sum * inv : 0.0, d.out_dtype);
        }
    }
}

template <int T>
void launch(hipStream_t stream, unsigned grid, int64_t per_block, size_t lds, const PreparedBatch& pb,
            const DeviceGraph& g, const MfmaTables& tab, const MfmaDims& d, const int64_t* item_begin, int64_t base,
            int64_t count, void* out, int64_t pitch, double* partial) {
    const bool general = d.weighted != 0 || d.radial != 0;
    auto kernel = d.radial != 0 ? k_soap_mfma<T, true, true> : general ? k_soap_mfma<T, true, false>
                                                                       : k_soap_mfma<T, false, false>;
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(T * kWaveThreads), lds, stream, pb.d_positions.as<double>(),
                       g.pair_start.as<int64_t>(), g.counts.as<int32_t>(), g.pair_bin.as<uint32_t>(), g.bin_x.as<double>(),
                       g.bin_y.as<double>(), g.bin_z.as<double>(), tab, tab.ps_pref, d, item_begin, base,
                       count, per_block, out, pitch, partial);
}

} // namespace

MfmaPlanHost plan_mfma_tables(int S, int n, int l_max, const std::vector<double>& beta_scaled,
                              const std::vector<double>& pref) {
    struct Block {
        int l, m_start, width;
    };
    struct Tile {
        int rows = 0, cols = 0;
        std::vector<int> ls;
    };
    std::vector<Block> blocks;
    for (int l = 0; l <= l_max; ++l) {
        const int c = 2 * l + 1;
        for (int start = 0; start < c; start += 16) blocks.push_back({l, start, std::min(16, c - start)});
    }
    std::stable_sort(blocks.begin(), blocks.end(), [](const Block& a, const Block& b) { return a.width > b.width; });
    std::vector<Tile> tiles;
    MfmaPlanHost out;
    std::vector<std::array<int, 3>> placed; // tile, row offset, col offset per block
    for (const Block& b : blocks) {
        int chosen = -1;
        for (size_t t = 0; t < tiles.size(); ++t) {
            const Tile& tile = tiles[t];
            const bool has_l = std::find(tile.ls.begin(), tile.ls.end(), b.l) != tile.ls.end();
            if (!has_l && tile.rows + n <= 16 && tile.cols + b.width <= 16) {
                chosen = static_cast<int>(t);
                break;
            }
        }
        if (chosen < 0) {
            tiles.emplace_back();
            chosen = static_cast<int>(tiles.size()) - 1;
        }
        Tile& tile = tiles[static_cast<size_t>(chosen)];
        placed.push_back({chosen, tile.rows, tile.cols});
        tile.rows += n;
        tile.cols += b.width;
        tile.ls.push_back(b.l);
    }
    const int T = static_cast<int>(tiles.size());
    out.tiles = T;
    out.row_channel.assign(static_cast<size_t>(T) * 16, -1);
    out.col_harmonic.assign(static_cast<size_t>(T) * 16, -1);
    for (size_t i = 0; i < blocks.size(); ++i) {
        const Block& b = blocks[i];
        const int t = placed[i][0], ro = placed[i][1], co = placed[i][2];
        for (int k = 0; k < n; ++k) out.row_channel[static_cast<size_t>(t * 16 + ro + k)] = b.l * n + k;
        for (int m = 0; m < b.width; ++m) {
            out.col_harmonic[static_cast<size_t>(t * 16 + co + m)] = b.l * b.l + b.m_start + m;
        }
    }
    out.beta_lane.assign(static_cast<size_t>(T) * 4 * 64, 0.0);
    for (int t = 0; t < T; ++t) {
        for (int s = 0; s < 4; ++s) {
            for (int lane = 0; lane < 64; ++lane) {
                const int row = lane % 16, kk = 4 * s + lane / 16;
                const int cr = out.row_channel[static_cast<size_t>(t * 16 + row)];
                const int ck = out.row_channel[static_cast<size_t>(t * 16 + kk)];
                if (cr >= 0 && ck >= 0 && cr / n == ck / n) {
                    const int l = cr / n, np = cr % n, k = ck % n;
                    out.beta_lane[static_cast<size_t>((t * 4 + s) * 64 + lane)] =
                        beta_scaled[static_cast<size_t>((l * n + np) * n + k)] * pref[static_cast<size_t>(ck)];
                }
            }
        }
    }
    // feature index of channel pair (i, j), i <= j: pair block (t1 <= t2) in
    // order, then l, then (n1, n2) with n2 >= n1 inside one species
    const int W = S * n, L = l_max + 1;
    out.fbase.assign(static_cast<size_t>(W) * W, -1);
    out.fstride.assign(static_cast<size_t>(W) * W, 0);
    int64_t base = 0;
    for (int t1 = 0; t1 < S; ++t1) {
        for (int t2 = t1; t2 < S; ++t2) {
            const int size = t1 == t2 ? n * (n + 1) / 2 : n * n;
            for (int n1 = 0; n1 < n; ++n1) {
                for (int n2 = (t1 == t2 ? n1 : 0); n2 < n; ++n2) {
                    const int inner = t1 == t2 ? n1 * n - n1 * (n1 - 1) / 2 + (n2 - n1) : n1 * n + n2;
                    const size_t idx = static_cast<size_t>((t1 * n + n1) * W + (t2 * n + n2));
                    out.fbase[idx] = static_cast<int32_t>(base + inner);
                    out.fstride[idx] = size;
                }
            }
            base += static_cast<int64_t>(L) * size;
        }
    }
    return out;
}

int mfma_template_tiles(int tiles) {
    static const int sizes[] = {1, 2, 3, 4, 6, 8, 12, 16};
    for (int s : sizes) {
        if (tiles <= s) return s;
    }
    return -1;
}

int mfma_padded_row(int l_max) {
    int off = 0;
    for (int l = 0; l <= l_max; ++l) off += 4 * ((2 * l + 4) / 4);
    // row stride = 4 (mod 32) doubles: the 16 rows x 4 columns that one
    // Gram-tile MFMA operand reads (and the 4 x 16 of the fold's stores) then
    // fall on distinct LDS banks in the fewest passes, for 32 or 64 banks
    return off + ((4 - off) % 32 + 32) % 32;
}

size_t mfma_lds_bytes(const MfmaDims& d) {
    const size_t cw = static_cast<size_t>(d.crow) * static_cast<size_t>(d.hpad);
    size_t words = static_cast<size_t>(kNb) * ((d.H + 1) | 1) + kNb + 64 + cw;
    if (d.mode == 1) words += cw;
    if (d.radial == 1) words += static_cast<size_t>(kNb) * (d.L * d.n + 1) + static_cast<size_t>(d.L) * kNb * 4;
    return words * sizeof(double) + static_cast<size_t>(d.L + 1 + 2 * (d.S + 1) + 1) * sizeof(int);
}

void launch_mfma_expand(hipStream_t stream, int template_tiles, const PreparedBatch& pb, const DeviceGraph& g,
                        const MfmaTables& tab, const MfmaDims& d, const int64_t* item_begin, int64_t base,
                        int64_t count, void* out, int64_t pitch, double* partial) {
    const size_t lds = mfma_lds_bytes(d);
    // split the harmonic m-columns over the workgroup's wavefronts, longest
    // recurrence (l_max - m + 1 values) first onto the least-loaded one
    MfmaDims dm = d;
    dm.cpitch = d.hpad;
    {
        int load[16] = {};
        for (int w = 0; w < 16; ++w) dm.harm_mask[w] = 0;
        for (int m = 0; m <= d.l_max; ++m) {
            int best = 0;
            for (int w = 1; w < template_tiles; ++w) {
                if (load[w] < load[best]) best = w;
            }
            dm.harm_mask[best] |= 1u << m;
            load[best] += d.l_max - m + 1;
        }
    }
    // persistent blocks: about two per wave slot the LDS footprint allows on
    // every CU, each walking a contiguous range of items
    const int64_t resident = std::max<int64_t>(1, std::min<int64_t>(32, (160 * 1024) / std::max<size_t>(lds, 1)));
    // a few centres per block: enough to amortise the block's table set-up,
    // few enough that the last blocks do not leave CUs idle
    const int64_t target = std::max<int64_t>(1, 8 * resident * device_compute_units());
    const int64_t per_block = std::max<int64_t>(1, (count + target - 1) / target);
    const unsigned grid = static_cast<unsigned>((count + per_block - 1) / per_block);
    if (count <= 0) return;
    switch (template_tiles) {
    case 1: launch<1>(stream, grid, per_block, lds, pb, g, tab, dm, item_begin, base, count, out, pitch, partial); break;
    case 2: launch<2>(stream, grid, per_block, lds, pb, g, tab, dm, item_begin, base, count, out, pitch, partial); break;
    case 3: launch<3>(stream, grid, per_block, lds, pb, g, tab, dm, item_begin, base, count, out, pitch, partial); break;
    case 4: launch<4>(stream, grid, per_block, lds, pb, g, tab, dm, item_begin, base, count, out, pitch, partial); break;
    case 6: launch<6>(stream, grid, per_block, lds, pb, g, tab, dm, item_begin, base, count, out, pitch, partial); break;
    case 8: launch<8>(stream, grid, per_block, lds, pb, g, tab, dm, item_begin, base, count, out, pitch, partial); break;
    case 12: launch<12>(stream, grid, per_block, lds, pb, g, tab, dm, item_begin, base, count, out, pitch, partial); break;
    case 16: launch<16>(stream, grid, per_block, lds, pb, g, tab, dm, item_begin, base, count, out, pitch, partial); break;
    default: throw Error(MDX_INTERNAL, "unsupported MFMA tile count");
    }
    MDX_HIP(hipGetLastError());
}

void launch_mfma_finalize(hipStream_t stream, const PreparedBatch& pb, const MfmaTables& tab, const MfmaDims& d,
                          const double* partial, const int64_t* struct_items, void* out, int64_t pitch) {
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>(pb.structures, 1 << 20));
    if (d.mode == 1) {
        // the partial rows are mean coefficients at a pitch of hpad
        MfmaDims dm = d;
        dm.cpitch = d.hpad;
        const size_t lds = static_cast<size_t>(d.crow) * d.hpad * sizeof(double)
            + static_cast<size_t>(d.L + 2) * sizeof(int);
        hipLaunchKernelGGL(k_mfma_finalize_inner, dim3(grid), dim3(kWaveThreads), lds, stream, partial, struct_items,
                           pb.d_offsets.as<int64_t>(), pb.structures, tab, dm, out, pitch);
    } else {
        hipLaunchKernelGGL(k_mfma_finalize_outer, dim3(grid), dim3(256), 0, stream, partial, struct_items,
                           pb.d_offsets.as<int64_t>(), pb.structures, d, out, pitch);
    }
    MDX_HIP(hipGetLastError());
}

} // namespace mdx
