// Kernels 2-4 on the FP64 matrix cores of gfx950 (v_mfma_f64_16x16x4f64).
//
// One wavefront owns one centre (or one run of centres of a structure for
// the "inner"/"outer" averages).  Per species segment of the centre's
// neighbour list (rows of kernel 1 are grouped by species):
//
//   contraction  A[(l,k)][(l,m)] = sum_j R_lk(j) Y_lm(j)      (soap.cpp:902-914)
//     The (l,k) x (l,m) products are packed block-diagonally into 16x16
//     tiles (rows = radial channels, columns = harmonics, several l per
//     tile); each MFMA adds 4 neighbours (K = 4).  A lane feeds the radial
//     value of its own tile row for every tile, so every exp(-a d^2) is
//     evaluated once, in the lane that consumes it; harmonics are computed
//     four lanes per neighbour by m-columns and staged in LDS.
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
#include "mdx_internal.h"
#include "soap_mfma.h"

#include <algorithm>
#include <array>
#include <cmath>

namespace mdx {

namespace {

typedef double d4 __attribute__((ext_vector_type(4)));

constexpr int kNb = 16;        // neighbours staged per chunk (4 MFMA steps)
constexpr int kWaveThreads = 64;

// Workgroups of the expansion kernel are a single wavefront: LDS operations
// of one wave complete in issue order, so cross-lane LDS hand-offs need only
// a compiler barrier and a wavefront-scope fence -- unlike __syncthreads(),
// which would also wait for the outstanding global prefetch.
__device__ inline void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ inline d4 mfma(double a, double b, d4 c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

__constant__ double c_inv_small[32] = {
    0.0, 1.0, 1.0 / 2, 1.0 / 3, 1.0 / 4, 1.0 / 5, 1.0 / 6, 1.0 / 7, 1.0 / 8, 1.0 / 9, 1.0 / 10,
    1.0 / 11, 1.0 / 12, 1.0 / 13, 1.0 / 14, 1.0 / 15, 1.0 / 16, 1.0 / 17, 1.0 / 18, 1.0 / 19, 1.0 / 20,
    1.0 / 21, 1.0 / 22, 1.0 / 23, 1.0 / 24, 1.0 / 25, 1.0 / 26, 1.0 / 27, 1.0 / 28, 1.0 / 29, 1.0 / 30,
    1.0 / 31};

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

// Harmonics of one neighbour for the m-columns m = m0, m0 + 4, ... (one of
// four cooperating lanes), written to a row of H values (entry (l, m') at
// l*l + m', m' = l -/+ m for cos/sin, the layout of soap.cpp:60-69).  Same
// recurrence as the generic kernel:
// (l-m) R_l^m = (2l-1) z R_{l-1}^m - (l+m-1) r^2 R_{l-2}^m, seeded by the
// Condon-Shortley diagonal (x + iy)^m (2m-1)!! (-1)^m.
__device__ void harmonic_columns(double x, double y, double z, int l_max, int L, int m0, const double* norm,
                                 double* out) {
    const double r2 = x * x + y * y + z * z;
    double re_mm = 1.0, im_mm = 0.0;
    int m_done = 0;
    for (int m = m0; m <= l_max; m += 4) {
        for (int q = m_done + 1; q <= m; ++q) {
            const double f = -(2.0 * q - 1.0);
            const double nr = f * (x * re_mm - y * im_mm);
            const double ni = f * (x * im_mm + y * re_mm);
            re_mm = nr;
            im_mm = ni;
        }
        m_done = m;
        double re2 = 0.0, im2 = 0.0, re1 = re_mm, im1 = im_mm;
        for (int l = m; l <= l_max; ++l) {
            double re0, im0;
            if (l == m) {
                re0 = re_mm;
                im0 = im_mm;
            } else if (l == m + 1) {
                re0 = (2.0 * m + 1.0) * z * re_mm;
                im0 = (2.0 * m + 1.0) * z * im_mm;
            } else {
                const double a = 2.0 * l - 1.0;
                const double b = (l + m - 1.0) * r2;
                const double inv = c_inv_small[l - m];
                re0 = (a * z * re1 - b * re2) * inv;
                im0 = (a * z * im1 - b * im2) * inv;
            }
            if (l > m) {
                re2 = re1;
                im2 = im1;
                re1 = re0;
                im1 = im0;
            }
            const double nf = norm[l * L + m];
            double* row = out + l * l;
            row[l - m] = nf * re0;
            if (m > 0) row[l + m] = nf * im0;
        }
    }
}

__device__ inline int degree_of_harmonic(int h) {
    int l = 0;
    while ((l + 1) * (l + 1) <= h) ++l;
    return l;
}

__device__ inline void store_out(void* out, int64_t pitch, int64_t row, int64_t f, double v, int dtype) {
    char* base = static_cast<char*>(out) + row * pitch;
    if (dtype == 4) {
        reinterpret_cast<float*>(base)[f] = static_cast<float>(v);
    } else {
        reinterpret_cast<double*>(base)[f] = v;
    }
}

// Feature index of channel pair (i, j), i <= j, at l = 0, and its stride
// per degree l, in the layout of soap.cpp:997-1013: species pairs t1 <= t2 in
// order, each a block of L x (n(n+1)/2) (t1 == t2, n2 >= n1) or L x n^2
// values ordered l, n1, n2.  Channel i is species i / n, radial i % n.
__device__ inline int feature_index(int i, int j, int S, int n, int L, int& stride) {
    const int t1 = i / n, n1 = i - t1 * n;
    const int t2 = j / n, n2 = j - t2 * n;
    const int same = n * (n + 1) / 2, cross = n * n;
    // blocks of the species rows a < t1, then (t1, t1 .. t2-1)
    int before = t1 * same + cross * (t1 * (S - 1) - t1 * (t1 - 1) / 2);
    if (t2 > t1) before += same + (t2 - t1 - 1) * cross;
    int inner;
    if (t1 == t2) {
        inner = n1 * n - n1 * (n1 - 1) / 2 + (n2 - n1);
        stride = same;
    } else {
        inner = n1 * n + n2;
        stride = cross;
    }
    return L * before + inner;
}

// Power spectrum of the coefficients in LDS on 16x16 Gram tiles.  s_c holds
// W + 1 rows of d.hpad values (row W and every pad entry are zero), entry
// (row, l, m') at row*hpad + loff[l] + m'.  mode 0: write row `row` of out;
// mode 2: add into the partial row `acc`.
__device__ void power_spectrum_tiles(const double* s_c, const int* loff, const MfmaDims& d, const double* ps_pref,
                                     int mode, void* out, int64_t pitch, int64_t row, double* acc) {
    const int lane = threadIdx.x;
    const int W = d.S * d.n;
    const int RT = (W + 15) / 16;
    const int hp = d.hpad;
    char* out_row = static_cast<char*>(out) + row * pitch;
    for (int bi = 0; bi < RT; ++bi) {
        for (int bj = bi; bj < RT; ++bj) {
            const int ia = min(16 * bi + lane % 16, W);
            const int jb = min(16 * bj + lane % 16, W);
            const double* arow = s_c + ia * hp + lane / 16;
            const double* brow = s_c + jb * hp + lane / 16;
            const int j = 16 * bj + lane % 16;
            int fb[4], fs[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = 16 * bi + lane / 16 + 4 * r;
                const bool ok = i < W && j < W && i <= j;
                fs[r] = 0;
                fb[r] = ok ? feature_index(i, j, d.S, d.n, d.L, fs[r]) : -1;
            }
            for (int l = 0; l <= d.l_max; ++l) {
                const int steps = (2 * l + 4) / 4;
                const int base = loff[l];
                d4 acc4 = {0.0, 0.0, 0.0, 0.0};
                for (int s = 0; s < steps; ++s) acc4 = mfma(arow[base + 4 * s], brow[base + 4 * s], acc4);
                const double pref = ps_pref[l];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (fb[r] >= 0) {
                        const int f = fb[r] + l * fs[r];
                        const double v = pref * acc4[r];
                        if (mode != 0) {
                            acc[f] += v;
                        } else if (d.out_dtype == 4) {
                            reinterpret_cast<float*>(out_row)[f] = static_cast<float>(v);
                        } else {
                            reinterpret_cast<double*>(out_row)[f] = v;
                        }
                    }
                }
            }
        }
    }
}

template <int T>
__global__ __launch_bounds__(kWaveThreads) void k_soap_mfma(
    const double* __restrict__ positions, const int64_t* __restrict__ pair_start, const int32_t* __restrict__ counts,
    const uint32_t* __restrict__ pair_bin, const double* __restrict__ bx, const double* __restrict__ by,
    const double* __restrict__ bz, const MfmaTables tab, MfmaDims d, const int64_t* __restrict__ item_begin,
    int64_t item_base, int64_t items, int64_t per_block, void* out, int64_t pitch, double* partial) {
    extern __shared__ double lds[];
    const int lane = threadIdx.x;
    const int H = d.H, L = d.L, S = d.S, n = d.n;
    const int W = S * n;
    const int HP = H + 1;                 // Y row stride; entry H stays zero
    const int hp = d.hpad;                // padded c row
    const int cw = (W + 1) * hp;          // c words, including the zero row W
    double* s_y = lds;                    // kNb * HP
    double* s_d2 = s_y + kNb * HP;        // kNb
    double* s_norm = s_d2 + kNb;          // L * L
    double* s_tab = s_norm + L * L;       // 64: 2^(j/64) for exp_neg
    double* s_c = s_tab + 64;             // cw (coefficients of the current centre, padded)
    double* s_csum = s_c + cw;            // cw (inner average only)
    int* s_loff = reinterpret_cast<int*>(s_csum + (d.mode == 1 ? cw : 0)); // L + 1
    int* s_seg = s_loff + (L + 1);        // S + 1: first row of each species segment of the centre

    for (int i = lane; i < L * L; i += kWaveThreads) s_norm[i] = tab.hnorm[i];
    s_tab[lane] = exp2(static_cast<double>(lane) / 64.0);
    for (int i = lane; i < kNb * HP; i += kWaveThreads) s_y[i] = 0.0;
    for (int i = lane; i < cw; i += kWaveThreads) s_c[i] = 0.0;
    if (lane == 0) {
        int off = 0;
        for (int l = 0; l <= L; ++l) {
            s_loff[l] = off;
            off += 4 * ((2 * l + 4) / 4);
        }
    }
    // per-lane tile constants: radial parameters of row lane%16 (zero for pad
    // rows, so their operand is 0 * e^0), Y column of lane%16 (the zero entry
    // H for pad columns), and the beta-fold destination of result row
    // lane/16 + 4r (or -1 off the diagonal blocks)
    int ycol[T];
    double pref[T], expo[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int rc = tab.row_channel[t * 16 + lane % 16];
        const int ch = tab.col_harmonic[t * 16 + lane % 16];
        ycol[t] = ch >= 0 ? ch : H;
        pref[t] = rc >= 0 ? tab.pref[rc] : 0.0;
        expo[t] = rc >= 0 ? tab.expo[rc] : 0.0;
    }
    wave_sync();
    int dst[T][4];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int ch = tab.col_harmonic[t * 16 + lane % 16];
        const int lh = ch >= 0 ? degree_of_harmonic(ch) : -1;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int och = tab.row_channel[t * 16 + lane / 16 + 4 * r];
            const bool diag = och >= 0 && ch >= 0 && och / n == lh;
            dst[t][r] = diag ? (och % n) * hp + s_loff[lh] + (ch - lh * lh) : -1;
        }
    }
    // A operands of the beta fold, the same for every species and centre
    double bfold[T][4];
#pragma unroll
    for (int t = 0; t < T; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) bfold[t][r] = tab.beta_lane[(t * 4 + r) * kWaveThreads + lane];
    }

    const int64_t item_first = item_base + static_cast<int64_t>(blockIdx.x) * per_block;
    const int64_t item_last = min(item_first + per_block, item_base + items);
    for (int64_t item = item_first; item < item_last; ++item) {
        const int64_t first = item_begin ? item_begin[item] : item;
        const int64_t last = item_begin ? item_begin[item + 1] : item + 1;
        double* part_row = partial != nullptr ? partial + item * (d.mode == 1 ? static_cast<int64_t>(cw) : d.F) : nullptr;
        if (d.mode == 1) {
            for (int i = lane; i < cw; i += kWaveThreads) s_csum[i] = 0.0;
        } else if (d.mode == 2) {
            for (int64_t i = lane; i < d.F; i += kWaveThreads) part_row[i] = 0.0;
        }
        for (int64_t centre = first; centre < last; ++centre) {
            const double cx = positions[centre * 3 + 0];
            const double cy = positions[centre * 3 + 1];
            const double cz = positions[centre * 3 + 2];
            const int64_t centre_pairs = pair_start[centre];
            // species segments of this centre's rows (kernel 1 groups them by species)
            if (lane == 0) {
                int rows = 0;
                for (int q = 0; q < S; ++q) {
                    s_seg[q] = rows;
                    rows += counts[centre * S + q];
                }
                s_seg[S] = rows;
            }
            wave_sync();
            // prefetch: lane (jj = lane/4) holds the image position of neighbour jj of the next chunk;
            // the first chunk starts at the centre's first row whatever its species
            double px = 0.0, py = 0.0, pz = 0.0;
            {
                const int jj = lane / 4;
                if (jj < min(kNb, s_seg[S])) {
                    const uint32_t b = pair_bin[centre_pairs + jj];
                    px = bx[b];
                    py = by[b];
                    pz = bz[b];
                }
            }
            for (int sp = 0; sp < S; ++sp) {
                const int seg0 = s_seg[sp];
                const int kt = s_seg[sp + 1] - seg0;
                if (kt == 0) {
                    // an empty species leaves its coefficients at zero
                    double* cdst = s_c + sp * n * hp;
                    for (int i = lane; i < n * hp; i += kWaveThreads) cdst[i] = 0.0;
                    continue;
                }
                d4 acc[T];
#pragma unroll
                for (int t = 0; t < T; ++t) acc[t] = d4{0.0, 0.0, 0.0, 0.0};
                for (int j0 = 0; j0 < kt; j0 += kNb) {
                    const int cnt = min(kNb, kt - j0);
                    wave_sync();
                    {
                        // four lanes per neighbour: geometry and m-columns of the harmonics;
                        // rows past the chunk's end are zeroed so they add nothing
                        const int jj = lane / 4;
                        const int sub = lane % 4;
                        double* yrow = s_y + jj * HP;
                        if (jj < cnt) {
                            // same arithmetic as kernel 1: image - centre, then d^2
                            const double dx = px - cx;
                            const double dy = py - cy;
                            const double dz = pz - cz;
                            if (sub == 0) s_d2[jj] = dx * dx + dy * dy + dz * dz;
                            harmonic_columns(dx, dy, dz, d.l_max, L, sub, s_norm, yrow);
                        } else {
                            if (sub == 0) s_d2[jj] = 0.0;
                            for (int h = sub; h < H; h += 4) yrow[h] = 0.0;
                        }
                    }
                    wave_sync();
                    {
                        // issue the loads of the next chunk now: rows are contiguous across
                        // species, so the next chunk starts right after this one, but a chunk
                        // never runs past its species' end
                        const int next = seg0 + j0 + kNb < s_seg[sp + 1] ? seg0 + j0 + kNb : s_seg[sp + 1];
                        int end = s_seg[sp + 1];
                        if (next == end) {
                            // first non-empty species after this one (empty ones own no rows)
                            for (int q = sp + 1; q < S; ++q) {
                                if (s_seg[q + 1] > next) {
                                    end = s_seg[q + 1];
                                    break;
                                }
                            }
                        }
                        const int avail = end - next;
                        const int jj = lane / 4;
                        if (avail > 0 && jj < min(kNb, avail)) {
                            const uint32_t b = pair_bin[centre_pairs + next + jj];
                            px = bx[b];
                            py = by[b];
                            pz = bz[b];
                        }
                    }
#pragma unroll
                    for (int s = 0; s < kNb / 4; ++s) {
                        const int jj = 4 * s + lane / 16;
                        const double d2 = s_d2[jj];
                        const double* yrow = s_y + jj * HP;
#pragma unroll
                        for (int t = 0; t < T; ++t) {
                            const double a = pref[t] * exp_neg(-expo[t] * d2, s_tab);
                            acc[t] = mfma(a, yrow[ycol[t]], acc[t]);
                        }
                    }
                }
                // fold beta: c_T = Bbeta_T x A_T; step r uses the accumulator register r as B
                double* cdst = s_c + sp * n * hp;
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    d4 c = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
                    for (int r = 0; r < 4; ++r) c = mfma(bfold[t][r], acc[t][r], c);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if (dst[t][r] >= 0) cdst[dst[t][r]] = c[r];
                    }
                }
            }
            wave_sync();
            if (d.mode == 0) {
                power_spectrum_tiles(s_c, s_loff, d, tab.ps_pref, 0, out, pitch, centre, nullptr);
            } else if (d.mode == 1) {
                for (int i = lane; i < cw; i += kWaveThreads) s_csum[i] += s_c[i];
            } else {
                power_spectrum_tiles(s_c, s_loff, d, tab.ps_pref, 2, out, pitch, centre, part_row);
            }
            wave_sync();
        }
        if (d.mode == 1) {
            for (int i = lane; i < cw; i += kWaveThreads) part_row[i] = s_csum[i];
        }
        wave_sync();
    }
}

// inner average: mean coefficients of each structure, then one power spectrum
__global__ __launch_bounds__(kWaveThreads) void k_mfma_finalize_inner(const double* partial, const int64_t* struct_items,
                                                                     const int64_t* offsets, int64_t structures,
                                                                     const MfmaTables tab, MfmaDims d, void* out,
                                                                     int64_t pitch) {
    extern __shared__ double lds[];
    const int W = d.S * d.n;
    const int cw = (W + 1) * d.hpad;
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
        power_spectrum_tiles(s_c, s_loff, d, tab.ps_pref, 0, out, pitch, s, nullptr);
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
    hipLaunchKernelGGL((k_soap_mfma<T>), dim3(grid), dim3(kWaveThreads), lds, stream, pb.d_positions.as<double>(),
                       g.pair_start.as<int64_t>(), g.counts.as<int32_t>(), g.pair_bin.as<uint32_t>(), g.bin_x.as<double>(),
                       g.bin_y.as<double>(), g.bin_z.as<double>(), tab, d, item_begin, base, count, per_block, out, pitch,
                       partial);
}

// Compute units of the current device (queried once per process and device).
int device_compute_units() {
    static int cached[64] = {};
    int dev = 0;
    MDX_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int cus = 0;
        MDX_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        cached[dev] = cus > 0 ? cus : 256;
    }
    return cached[dev];
}

} // namespace

MfmaPlanHost plan_mfma_tables(int S, int n, int l_max, const std::vector<double>& beta_scaled) {
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
                        beta_scaled[static_cast<size_t>((l * n + np) * n + k)];
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
    return off;
}

size_t mfma_lds_bytes(const MfmaDims& d) {
    const size_t W = static_cast<size_t>(d.S) * d.n;
    const size_t cw = (W + 1) * static_cast<size_t>(d.hpad);
    size_t words = static_cast<size_t>(kNb) * (d.H + 1) + kNb + static_cast<size_t>(d.L) * d.L + 64 + cw;
    if (d.mode == 1) words += cw;
    return words * sizeof(double) + static_cast<size_t>(d.L + 1 + kMaxSpecies + 1) * sizeof(int);
}

void launch_mfma_expand(hipStream_t stream, int template_tiles, const PreparedBatch& pb, const DeviceGraph& g,
                        const MfmaTables& tab, const MfmaDims& d, const int64_t* item_begin, int64_t base,
                        int64_t count, void* out, int64_t pitch, double* partial) {
    const size_t lds = mfma_lds_bytes(d);
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
    case 1: launch<1>(stream, grid, per_block, lds, pb, g, tab, d, item_begin, base, count, out, pitch, partial); break;
    case 2: launch<2>(stream, grid, per_block, lds, pb, g, tab, d, item_begin, base, count, out, pitch, partial); break;
    case 3: launch<3>(stream, grid, per_block, lds, pb, g, tab, d, item_begin, base, count, out, pitch, partial); break;
    case 4: launch<4>(stream, grid, per_block, lds, pb, g, tab, d, item_begin, base, count, out, pitch, partial); break;
    case 6: launch<6>(stream, grid, per_block, lds, pb, g, tab, d, item_begin, base, count, out, pitch, partial); break;
    case 8: launch<8>(stream, grid, per_block, lds, pb, g, tab, d, item_begin, base, count, out, pitch, partial); break;
    case 12: launch<12>(stream, grid, per_block, lds, pb, g, tab, d, item_begin, base, count, out, pitch, partial); break;
    case 16: launch<16>(stream, grid, per_block, lds, pb, g, tab, d, item_begin, base, count, out, pitch, partial); break;
    default: throw Error(MDX_INTERNAL, "unsupported MFMA tile count");
    }
    MDX_HIP(hipGetLastError());
}

void launch_mfma_finalize(hipStream_t stream, const PreparedBatch& pb, const MfmaTables& tab, const MfmaDims& d,
                          const double* partial, const int64_t* struct_items, void* out, int64_t pitch) {
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>(pb.structures, 1 << 20));
    if (d.mode == 1) {
        const size_t lds = (static_cast<size_t>(d.S) * d.n + 1) * d.hpad * sizeof(double)
            + static_cast<size_t>(d.L + 2) * sizeof(int);
        hipLaunchKernelGGL(k_mfma_finalize_inner, dim3(grid), dim3(kWaveThreads), lds, stream, partial, struct_items,
                           pb.d_offsets.as<int64_t>(), pb.structures, tab, d, out, pitch);
    } else {
        hipLaunchKernelGGL(k_mfma_finalize_outer, dim3(grid), dim3(256), 0, stream, partial, struct_items,
                           pb.d_offsets.as<int64_t>(), pb.structures, d, out, pitch);
    }
    MDX_HIP(hipGetLastError());
}

} // namespace mdx
