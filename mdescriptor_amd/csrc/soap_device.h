// Device helpers shared by the matrix-core SOAP kernels (soap_mfma.hip,
// soap_quad.hip): MFMA wrappers, the real solid harmonics, the feature index
// of the power spectrum and the Gram-tile power-spectrum walk.  Everything is
// in an anonymous namespace: each translation unit gets its own copy.
#pragma once

#include "harmonic_table.h"
#include "mdx_internal.h"
#include "soap_mfma.h"

namespace mdx {
namespace {

typedef double d4 __attribute__((ext_vector_type(4)));

constexpr int kNb = 32;        // neighbours staged per chunk (8 MFMA steps)
constexpr int kWaveThreads = 64;

// 64-bit value of lane `src` (a compile-time lane) in scalar registers.
__device__ inline int64_t lane_value(int64_t v, int src) {
    const int lo = __builtin_amdgcn_readlane(static_cast<int>(v), src);
    const int hi = __builtin_amdgcn_readlane(static_cast<int>(v >> 32), src);
    return static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo));
}

__device__ inline d4 mfma(double a, double b, d4 c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

// Normalised real solid harmonics Q_l^m = N_lm R_l^m of one neighbour, one
// component per lane: comp 0 writes the cos parts (entry l*l + l - m), comp 1
// the sin parts (l*l + l + m, m > 0), the layout of soap.cpp:60-69, by the
// recurrences of harmonic_table.h.  Only the m-columns set in `mask` are
// computed (the workgroup's wavefronts split them).  With l_max = LM fixed at
// compile time both loops unroll completely: every coefficient is an
// immediate constant and every store a constant LDS offset from the lane's
// column base.  Entry h of the lane's slot sits at out[h * kStride].
template <int LM, int kStride = 1>
__device__ __forceinline__ void harmonics_fixed(double x, double y, double z, double scale, uint32_t mask, int comp,
                                               const HarmonicRecurrence* __restrict__ hr, double* out) {
    const double r2 = x * x + y * y + z * z;
    // the seed carries the neighbour's weight: every harmonic is linear in it,
    // and a pad slot (scale 0) gets all-zero harmonics
    double sre = scale * hr->n00, sim = 0.0;
#pragma unroll
    for (int m = 0; m <= LM; ++m) {
        if ((mask >> m) == 0) break;  // no column of this wavefront from here on
        if (m > 0) {
            const double dm = hr->d[m];
            const double nr = dm * fma(x, sre, -(y * sim));
            const double ni = dm * fma(x, sim, y * sre);
            sre = nr;
            sim = ni;
        }
        if (((mask >> m) & 1u) == 0) continue;
        double* col = out + (comp == 0 ? -m : m) * kStride; // entry (l, m) of this lane's part at col[(l*l + l) * kStride]
        double q1 = comp == 0 ? sre : sim;
        if (m > 0 || comp == 0) col[(m * m + m) * kStride] = q1;
        if (m + 1 > LM) continue;
        double q2 = q1;
        q1 = hr->e[m] * (z * q2);
        if (m > 0 || comp == 0) col[((m + 1) * (m + 1) + (m + 1)) * kStride] = q1;
#pragma unroll
        for (int l = m + 2; l <= LM; ++l) {
            const double q = fma(hr->a[l][m] * z, q1, -(hr->b[l][m] * r2) * q2);
            if (m > 0 || comp == 0) col[(l * l + l) * kStride] = q;
            q2 = q1;
            q1 = q;
        }
    }
}

// The same harmonics in the scaled form of harmonic_table.h: writes
// Qs_l^m = Q_l^m / S_lm (the caller applies S_lm to whatever it accumulates
// from them).  Same lanes, masks and layout as harmonics_fixed.
template <int LM, int kStride>
__device__ __forceinline__ void harmonics_scaled_fixed(double x, double y, double z, double scale, uint32_t mask,
                                                      int comp, const ScaledHarmonicRecurrence* __restrict__ hr,
                                                      double* out) {
    const double r2 = x * x + y * y + z * z;
    double sre = scale, sim = 0.0;
#pragma unroll
    for (int m = 0; m <= LM; ++m) {
        if ((mask >> m) == 0) break;
        if (m > 0) {
            const double nr = fma(x, sre, -(y * sim));
            const double ni = fma(x, sim, y * sre);
            sre = nr;
            sim = ni;
        }
        if (((mask >> m) & 1u) == 0) continue;
        double* col = out + (comp == 0 ? -m : m) * kStride;
        double q1 = comp == 0 ? sre : sim;
        if (m > 0 || comp == 0) col[(m * m + m) * kStride] = q1;
        if (m + 1 > LM) continue;
        double q2 = q1;
        q1 = z * q2;
        if (m > 0 || comp == 0) col[((m + 1) * (m + 1) + (m + 1)) * kStride] = q1;
#pragma unroll
        for (int l = m + 2; l <= LM; ++l) {
            const double q = fma(z, q1, -(hr->c[l][m] * r2) * q2);
            if (m > 0 || comp == 0) col[(l * l + l) * kStride] = q;
            q2 = q1;
            q1 = q;
        }
    }
}

template <int LM = 0, int kTop = kHarmonicLmax, int kStride = 1>
__device__ __forceinline__ void harmonics_scaled(double x, double y, double z, double scale, int l_max, uint32_t mask,
                                                int comp, const ScaledHarmonicRecurrence* __restrict__ hr,
                                                double* out) {
    if (l_max == LM) {
        harmonics_scaled_fixed<LM, kStride>(x, y, z, scale, mask, comp, hr, out);
    } else if constexpr (LM < kTop) {
        harmonics_scaled<LM + 1, kTop, kStride>(x, y, z, scale, l_max, mask, comp, hr, out);
    }
}

// harmonics_fixed<l_max, kStride> for a run-time l_max <= kTop (a wave-uniform
// branch chain)
template <int LM = 0, int kTop = kHarmonicLmax, int kStride = 1>
__device__ __forceinline__ void harmonics_q(double x, double y, double z, double scale, int l_max, uint32_t mask,
                                           int comp, const HarmonicRecurrence* __restrict__ hr, double* out) {
    if (l_max == LM) {
        harmonics_fixed<LM, kStride>(x, y, z, scale, mask, comp, hr, out);
    } else if constexpr (LM < kTop) {
        harmonics_q<LM + 1, kTop, kStride>(x, y, z, scale, l_max, mask, comp, hr, out);
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

// i / n for 0 <= i < 256, 1 <= n <= 16 without an integer division:
// (i + 1/2) / n sits at least 1/32 away from an integer, far beyond the
// float rounding of the product.
__device__ inline int div_small(int i, float inv_n) {
    return static_cast<int>((static_cast<float>(i) + 0.5f) * inv_n);
}

// Feature index of channel pair (i, j), i <= j, at l = 0, and its stride
// per degree l, in the layout of soap.cpp:997-1013: species pairs t1 <= t2 in
// order, each a block of L x (n(n+1)/2) (t1 == t2, n2 >= n1) or L x n^2
// values ordered l, n1, n2.  Channel i is species i / n, radial i % n.
__device__ inline int feature_index(int i, int j, int S, int n, float inv_n, int L, int& stride) {
    const int t1 = div_small(i, inv_n), n1 = i - t1 * n;
    const int t2 = div_small(j, inv_n), n2 = j - t2 * n;
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

// mu1nu1: rows W + n2 of s_c = sum over species of rows t n + n2 (the
// summed density of soap.cpp:955-967).  All threads of the workgroup; the
// caller synchronises before the power spectrum reads them.
__device__ void species_sums(double* s_c, const MfmaDims& d, int tid, int threads) {
    const int n = d.n, hp = d.cpitch, W = d.Sc * n;
    for (int i = tid; i < n * hp; i += threads) {
        const int n2 = i / hp, e = i - n2 * hp;
        double sum = 0.0;
        for (int t = 0; t < d.Sc; ++t) sum += s_c[(t * n + n2) * hp + e];
        s_c[(W + n2) * hp + e] = sum;
    }
}

// Power spectrum of the coefficients in LDS on 16x16 Gram tiles.  s_c holds
// W + 1 rows of d.hpad values at a pitch of d.cpitch (row W and every pad
// entry are zero), entry (row, l, m') at row*cpitch + loff[l] + m'.  The units (tile pair, l), pair-
// major, are split into contiguous ranges over the `waves` wavefronts of the
// workgroup (wavefront `wave` takes its range); units write disjoint
// features, and a given feature always comes from the same wavefront.
// mode 0: write row `row` of out; mode 2: add into the partial row `acc`;
// mode 3: store into `acc` (the first centre of a run).
//
// Compression (soap.cpp:948-996): "mu2" has one coefficient species, so it is
// the plain layout with Sc = 1; "crossover" keeps the pairs inside a species;
// "mu1nu1" pairs every channel (t, n1) with the species-summed row n2 (rows W
// .. W+n-1 of s_c, filled by species_sums), over all (n1, n2).
// kPaired: mu1nu1 or crossover; the plain walk (off, mu2) is compiled without
// their branches.
template <bool kPaired>
__device__ void power_spectrum_walk(const double* s_c, const int* loff, const MfmaDims& d,
                                    const double* __restrict__ ps_pref, int mode, void* out, int64_t pitch,
                                    int64_t row, double* acc, int wave, int waves) {
    const int lane = threadIdx.x % kWaveThreads;
    const int W = d.Sc * d.n;
    const int zero_row = d.crow - 1;
    const int RT = (W + 15) / 16;
    const bool rect = kPaired && d.compression == 2; // A = channels, B = summed rows
    const int RB = rect ? (d.n + 15) / 16 : RT;
    const int L = d.L;
    const int hp = d.cpitch;
    const int n = d.n;
    const float inv_n = 1.0f / static_cast<float>(n);
    const int units = (rect ? RT * RB : RT * (RT + 1) / 2) * L;
    const int u_begin = wave * units / waves;
    const int u_end = (wave + 1) * units / waves;
    if (u_begin >= u_end) return;
    char* out_row = static_cast<char*>(out) + row * pitch;
    // first unit of the range: pair p = (bi, bj), bi <= bj, row-major over the
    // upper triangle of tile pairs, and degree l; later units step l, then bj, then bi
    int p = u_begin / L;
    int l = u_begin - p * L;
    int bi = 0, bj = 0;
    if (rect) {
        bi = p / RB;
        bj = p - bi * RB;
    } else {
        while (p >= RT - bi) {
            p -= RT - bi;
            ++bi;
        }
        bj = bi + p;
    }
    const double* arow = s_c;
    const double* brow = s_c;
    int fb[4] = {-1, -1, -1, -1}, fs[4] = {0, 0, 0, 0};
    bool new_pair = true;
    for (int u = u_begin; u < u_end; ++u) {
        if (new_pair) {
            new_pair = false;
            const int ia = 16 * bi + lane % 16 < W ? 16 * bi + lane % 16 : zero_row;
            const int jrow = rect ? W + 16 * bj + lane % 16 : 16 * bj + lane % 16;
            const int jlim = rect ? W + n : W;
            const int jb = jrow < jlim ? jrow : zero_row;
            arow = s_c + ia * hp + lane / 16;
            brow = s_c + jb * hp + lane / 16;
            const int j = 16 * bj + lane % 16;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = 16 * bi + lane / 16 + 4 * r;
                fs[r] = 0;
                fb[r] = -1;
                if (rect) {
                    // mu1nu1: i = t n + n1 against summed row j = n2 (soap.cpp:969-981)
                    if (i < W && j < n) {
                        const int t = div_small(i, inv_n);
                        fs[r] = n * n;
                        fb[r] = t * L * n * n + (i - t * n) * n + j;
                    }
                } else if (i < W && j < W && i <= j) {
                    if (kPaired && d.compression == 3) {
                        // crossover: same species only (soap.cpp:983-995)
                        const int t1 = div_small(i, inv_n), t2 = div_small(j, inv_n);
                        if (t1 == t2) {
                            const int n1 = i - t1 * n, n2 = j - t2 * n;
                            const int same = n * (n + 1) / 2;
                            fs[r] = same;
                            fb[r] = t1 * L * same + n1 * n - n1 * (n1 - 1) / 2 + (n2 - n1);
                        }
                    } else {
                        fb[r] = feature_index(i, j, d.Sc, n, inv_n, L, fs[r]);
                    }
                }
            }
        }
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
                if (mode == 2) {
                    acc[f] += v;
                } else if (mode == 3) {
                    acc[f] = v;
                } else if (d.out_dtype == 4) {
                    reinterpret_cast<float*>(out_row)[f] = static_cast<float>(v);
                } else {
                    reinterpret_cast<double*>(out_row)[f] = v;
                }
            }
        }
        if (++l == L) {
            l = 0;
            new_pair = true;
            if (rect) {
                if (++bj == RB) {
                    ++bi;
                    bj = 0;
                }
            } else if (++bj == RT) {
                ++bi;
                bj = bi;
            }
        }
    }
}

__device__ inline void power_spectrum_tiles(const double* s_c, const int* loff, const MfmaDims& d,
                                            const double* __restrict__ ps_pref, int mode, void* out, int64_t pitch,
                                            int64_t row, double* acc, int wave, int waves) {
    if (d.compression >= 2) {
        power_spectrum_walk<true>(s_c, loff, d, ps_pref, mode, out, pitch, row, acc, wave, waves);
    } else {
        power_spectrum_walk<false>(s_c, loff, d, ps_pref, mode, out, pitch, row, acc, wave, waves);
    }
}

constexpr double kPi = 3.141592653589793238462643383279502884;

// x^m: a whole exponent of at most 32 in magnitude by binary powering (at
// most ten products, for the usual 2 to 12 a few), any other through pow
__device__ inline double weight_power(double x, double m) {
    const double whole = rint(m);
    if (whole != m || fabs(m) > 32.0) return pow(x, m);
    int e = static_cast<int>(fabs(m));
    double base = x, result = 1.0;
    while (e != 0) {
        if (e & 1) result *= base;
        e >>= 1;
        if (e != 0) base *= base;
    }
    return m < 0.0 ? 1.0 / result : result;
}

// Distance function of a neighbour's weight (soap_weight, soap.cpp:389-420):
// 1 poly, c (1 + 2x^3 - 3x^2)^m for x = r / r0 <= 1, else 0; 2 pow,
// c / (d + x^m); 3 exp, c / (d + e^-x); 0 none (1).
__device__ inline double weight_function(int kind, double r0, double c, double d, double m, double distance) {
    if (kind == 0) return 1.0;
    const double ratio = distance / r0;
    if (kind == 1) {
        return distance > r0 ? 0.0 : c * weight_power(1.0 + 2.0 * ratio * ratio * ratio - 3.0 * ratio * ratio, m);
    }
    if (kind == 2) return c / (d + weight_power(ratio, m));
    return c / (d + exp(-ratio));
}

} // namespace
} // namespace mdx
