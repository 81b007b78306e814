// Coefficients of the recurrence for the normalised real solid harmonics
//   Q_l^m = N_lm r^l P_l^m(cos t) {cos, sin}(m phi),
//   N_lm = sqrt((2l+1)/(4 pi) (l-m)!/(l+m)!) (times sqrt(2) for m > 0),
// the quantity of soap.cpp:26-38 and :60-69, generated at compile time so
// that kernels unrolled over (l, m) see them as immediate constants:
//   Q_0^0 = N_00 = 1 / (2 sqrt(pi))
//   Q_m^m = D_m (x + iy) Q_{m-1}^{m-1},  D_m = -sqrt((2m+1)/(2m)) (times sqrt(2) at m = 1)
//   Q_{m+1}^m = E_m z Q_m^m,             E_m = sqrt(2m+3)
//   Q_l^m = A_lm z Q_{l-1}^m - B_lm r^2 Q_{l-2}^m,
//     A_lm = sqrt((2l-1)(2l+1) / ((l-m)(l+m))),
//     B_lm = sqrt((2l+1)(l+m-1)(l-m-1) / ((2l-3)(l-m)(l+m))).
// The last line is the associated-Legendre three-term recurrence in l with
// the ratios N_lm / N_{l-1,m} and N_lm / N_{l-2,m} folded in.
//
// Plain C++17 (no HIP types) so host code and tests can include it too.
#pragma once

namespace mdx {

constexpr int kHarmonicLmax = 20;

namespace detail {

// Dekker's split of a double into two 26-bit halves (exact products below).
constexpr double split_hi(double x) {
    const double c = 134217729.0 * x;  // 2^27 + 1
    return c - (c - x);
}

// x^2 - v, exact to well below ulp(v) for x near sqrt(v).
constexpr double square_residual(double x, double v) {
    const double hi = split_hi(x);
    const double lo = x - hi;
    return ((hi * hi - v) + 2.0 * hi * lo) + lo * lo;
}

constexpr double abs_value(double x) { return x < 0.0 ? -x : x; }

// sqrt(v) for v > 0 at compile time: Newton's iteration from above, then the
// neighbour (one unit in the last place either way) with the smallest
// residual |x^2 - v|, which is the correctly rounded root.
constexpr double ct_sqrt(double v) {
    if (!(v > 0.0)) return 0.0;
    double x = v > 1.0 ? v : 1.0;
    for (int i = 0; i < 2000; ++i) {
        const double next = 0.5 * (x + v / x);
        if (!(next < x)) break;
        x = next;
    }
    double best = x;
    double best_r = abs_value(square_residual(x, v));
    for (int k = 0; k < 2; ++k) {
        // ulp of x from its exponent, by scaling (no bit casts in constexpr)
        double ulp = 1.0;
        while (ulp * 4503599627370496.0 > x) ulp *= 0.5;  // 2^52 ulp <= x
        while (ulp * 9007199254740992.0 <= x) ulp *= 2.0; // x < 2^53 ulp
        const double candidates[2] = {best - ulp, best + ulp};
        double improved = best;
        for (double c : candidates) {
            const double r = abs_value(square_residual(c, v));
            if (r < best_r) {
                best_r = r;
                improved = c;
            }
        }
        if (improved == best) break;
        best = improved;
        x = best;
    }
    return best;
}

} // namespace detail

struct HarmonicRecurrence {
    double n00;
    double d[kHarmonicLmax + 1];
    double e[kHarmonicLmax + 1];
    double a[kHarmonicLmax + 1][kHarmonicLmax + 1];
    double b[kHarmonicLmax + 1][kHarmonicLmax + 1];
};

constexpr HarmonicRecurrence make_harmonic_recurrence() {
    HarmonicRecurrence t{};
    constexpr double pi = 3.14159265358979323846;
    t.n00 = 0.5 / detail::ct_sqrt(pi);
    for (int m = 1; m <= kHarmonicLmax; ++m) {
        const double dm = -detail::ct_sqrt((2.0 * m + 1.0) / (2.0 * m));
        t.d[m] = m == 1 ? dm * detail::ct_sqrt(2.0) : dm;
    }
    for (int m = 0; m < kHarmonicLmax; ++m) t.e[m] = detail::ct_sqrt(2.0 * m + 3.0);
    for (int l = 2; l <= kHarmonicLmax; ++l) {
        for (int m = 0; m + 2 <= l; ++m) {
            const double lm = static_cast<double>(l - m), lp = static_cast<double>(l + m);
            t.a[l][m] = detail::ct_sqrt((2.0 * l - 1.0) * (2.0 * l + 1.0) / (lm * lp));
            t.b[l][m] = detail::ct_sqrt((2.0 * l + 1.0) * (lp - 1.0) * (lm - 1.0) / ((2.0 * l - 3.0) * lm * lp));
        }
    }
    return t;
}

constexpr HarmonicRecurrence kHarmonic = make_harmonic_recurrence();

// Scaled form of the same recurrence, Q_l^m = S_lm Qs_l^m, with the scales
// chosen so that the z coefficient of every step is one:
//   Qs_m^m = (x + iy)^m Qs_0^0,  Qs_{m+1}^m = z Qs_m^m,
//   Qs_l^m = z Qs_{l-1}^m - C_lm r^2 Qs_{l-2}^m,
//   S_00 = N_00,  S_mm = D_m S_{m-1,m-1},  S_{m+1,m} = E_m S_mm,  S_lm = A_lm S_{l-1,m},
//   C_lm = B_lm S_{l-2,m} / S_lm.
// A step then costs one multiply-add and two multiplies; S_lm is applied once
// per coefficient instead of once per neighbour.
struct ScaledHarmonicRecurrence {
    double s[kHarmonicLmax + 1][kHarmonicLmax + 1]; // S_lm, m <= l
    double c[kHarmonicLmax + 1][kHarmonicLmax + 1]; // C_lm, m + 2 <= l
};

constexpr ScaledHarmonicRecurrence make_scaled_harmonic_recurrence() {
    ScaledHarmonicRecurrence t{};
    const HarmonicRecurrence h = make_harmonic_recurrence();
    t.s[0][0] = h.n00;
    for (int m = 1; m <= kHarmonicLmax; ++m) t.s[m][m] = h.d[m] * t.s[m - 1][m - 1];
    for (int m = 0; m < kHarmonicLmax; ++m) t.s[m + 1][m] = h.e[m] * t.s[m][m];
    for (int m = 0; m <= kHarmonicLmax; ++m) {
        for (int l = m + 2; l <= kHarmonicLmax; ++l) {
            t.s[l][m] = h.a[l][m] * t.s[l - 1][m];
            t.c[l][m] = h.b[l][m] * t.s[l - 2][m] / t.s[l][m];
        }
    }
    return t;
}

constexpr ScaledHarmonicRecurrence kScaledHarmonic = make_scaled_harmonic_recurrence();

} // namespace mdx
