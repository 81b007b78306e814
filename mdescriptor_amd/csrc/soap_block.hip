// Kernels 2-4 for the default SOAP options (GTO basis, no weighting, no
// compression) with the coefficients held in registers: neighbour expansion
// on 4x4x4 FP64 matrix-core blocks, beta fold, power spectrum on 16x16x4 FP64
// Gram tiles and the row write (soap.cpp:864-930, 997-1013).
//
// One workgroup of T wavefronts handles one centre at a time.  Degree l is
// owned by one wavefront, which keeps everything of that degree in its
// registers: the contraction accumulators, the coefficients of every species
// and the power spectrum.  The wavefronts share only the harmonic staging in
// LDS, double-buffered, with one barrier per chunk of 32 neighbour slots.
//
// Matrix-core layouts (v_mfma_f64_4x4x4f64, four independent 4x4 blocks; the
// block of lane L is b = (L/4) % 4):
//   A operand lane L = A_b[row L % 4][k L / 16]
//   B operand lane L = B_b[k L / 16][col L % 4]
//   result    lane L = D_b[row L / 16][col L % 4]
// and for v_mfma_f64_16x16x4f64: A lane L = A[row L % 16][k L / 16],
// B lane L = B[k L / 16][col L % 16], result value r of lane L =
// D[row 4 r + L / 16][col L % 16].
//
// Contraction, A[(l,k)][(l,m)] = sum_j e^{-a_lk d_j^2} Y_lm(j)
// (soap.cpp:893-914).  An exp register of degree l holds, per block, radial
// group rg (4 channels k) at step phase ph: R radial groups times P = 4/R
// phases (R = 2 for two radial groups, else 1), so one register of exps feeds
// P consecutive steps of 4 neighbours and no lane computes an exp that is not
// used.  Its MFMA with the harmonic block of column group cg (4 columns of
// degree l) accumulates blocks (rg, ph) x (k, m).  Each species' rows fill a
// segment of slots padded to a whole step group (4 P slots), so a group never
// mixes species.
//
// At a species change the phases of each accumulator are summed (row
// rotations) and the species' radial groups are added into the block slots of
// its "channel groups" (species q, radial group rg) of the coefficient
// registers C[r], r = group / 4, slot group % 4 (for three radial groups, one
// register per species, slot rg).  At the end of the centre every C[r] is
// scaled by the harmonic scale S_lm of its columns (the staged harmonics are
// the scaled recurrence of harmonic_table.h; pad columns have S_lm = 0) and
// folded with beta (soap.cpp:915-926) in transposed form,
//   c^T = A^T beta^T:  A operand = the accumulator (lane L = A[k L/16][m L%4]
//   read as A^T[m][k]), B operand = beta^T (lane constant),
// which leaves lane L of block (group) b holding c[n' = L % 4][m = L / 16]:
// exactly a 16x16x4 Gram operand whose 16 rows are 4 channel groups x 4 radial
// channels and whose K index is m.  The radial groups of a species mix through
// the fold terms: two radial groups exchange blocks b and b^1 (lane swizzle),
// three rotate the blocks of the species' register.
//
// Power spectrum (soap.cpp:997-1013): p_l[i][j] = sum_m c[i][m] c[j][m] for the
// degrees a wavefront owns, one 16x16x4 MFMA per column group and register
// pair, scaled by pi sqrt(8/(2l+1)) and stored with raw buffer stores whose
// range check drops the pairs i > j and the pad channels.
#include "soap_device.h"
#include "soap_block.h"

#include <algorithm>
#include <cmath>
#include <type_traits>
#include <utility>

namespace mdx {
namespace {

constexpr int kYS = kNb + 1;       // harmonic staging: entry h of slot j at h * kYS + j
constexpr int kTabBits = 8;
constexpr int kTab = 1 << kTabBits; // 2^(j/256) table entries
// Power-spectrum feature offsets are packed as (byte offset << 9) | feature
// stride per degree; a pair that is not stored gets kDroppedBytes, past the
// end of every row this kernel writes (the buffer range check drops the
// store).  Rows must be shorter than kDroppedBytes (checked on the host).
constexpr int kStrideBits = 9;
constexpr int kDroppedBytes = (1 << 22) - 1;

// square root of pi sqrt(8 / (2l + 1)), the power-spectrum prefactor
// (soap.cpp:513-516): each coefficient carries it, so the Gram product of two
// coefficient rows carries the prefactor
struct PsRoots {
    double v[kHarmonicLmax + 1];
};
constexpr PsRoots make_ps_roots() {
    PsRoots r{};
    for (int l = 0; l <= kHarmonicLmax; ++l)
        r.v[l] = detail::ct_sqrt(3.141592653589793238462643383279502884 * detail::ct_sqrt(8.0 / (2.0 * l + 1.0)));
    return r;
}
__device__ constexpr PsRoots kPsRootTable = make_ps_roots();
#define kPsRoot kPsRootTable.v

// ---------------------------------------------------------------- plan ----

constexpr int cgroups(int l) { return (2 * l + 4) / 4; } // ceil((2l+1)/4)

template <int LM, int KG>
struct BlockPlan {
    static constexpr int L = LM + 1;
    static constexpr int H = L * L;
    static constexpr int R = KG == 2 ? 2 : 1;   // radial groups per exp register
    static constexpr int P = 4 / R;             // step phases per exp register
    static constexpr int RPL = KG / R;          // exp registers per degree
    static constexpr int NT = KG == 1 ? 1 : KG == 2 ? 2 : 4; // fold terms
    static constexpr int GS = 4 * P;            // slots per step group
    static constexpr int GROUPS = kNb / GS;     // step groups per chunk
    static constexpr int T = L < 4 ? L : 4;     // wavefronts
    // staged harmonic rows; the pad columns of degree LM (up to 3) read
    // the rows that follow a buffer: the next buffer's first rows, or after
    // the second buffer the d2 and exp tables, all finite
    static constexpr int YROWS = H;
    static constexpr int YWORDS = YROWS * kYS;
    // wavefronts that stage the harmonics (the first HW roles): each pays a
    // per-slot set-up, so fewer of them do less work in total; from l_max 8
    // one wavefront's share of the columns outweighs it (measured: two
    // wavefronts 6 % faster at l_max 8 and 9, 7-11 % slower at 3, 4 and 6)
    static constexpr int HW = (LM >= 8 ? 2 : 1) < T ? (LM >= 8 ? 2 : 1) : T;
    // with one harmonic wavefront it owns no degree: its staging alone is
    // about as long as two degrees' exps, and the wavefronts of a workgroup
    // meet at a barrier every chunk (measured: 9-10 % faster at l_max 3 and
    // 4, 4 % at 6; with two harmonic wavefronts, l_max 8 and 9, the
    // remaining two would hold every degree: 40 % slower)
    static constexpr bool HO = HW == 1 && T > 1;

    // degrees of each wavefront: longest processing time first over the cost
    // of a degree per step group (exps of 12 VALU instructions, 4 cycles each,
    // and its MFMAs of 16 cycles), the harmonic wavefronts starting with
    // their share of the staging (their columns' VALU instructions per chunk,
    // 4 cycles each, spread over the chunk's step groups)
    struct Owners {
        unsigned mask[4];
    };
    static constexpr Owners owners() {
        Owners o{};
        int load[4] = {0, 0, 0, 0};
        for (int w = 0; w < HW; ++w) load[w] = HO ? (1 << 20) : 4 * range_cost(mlo(w), mhi(w)) / GROUPS;
        bool done[L] = {};
        for (int it = 0; it < L; ++it) {
            int best = -1, best_cost = -1;
            for (int l = L - 1; l >= 0; --l) {
                const int c = RPL * (48 + 16 * cgroups(l));
                if (!done[l] && c > best_cost) {
                    best = l;
                    best_cost = c;
                }
            }
            done[best] = true;
            int w = 0;
            for (int v = 1; v < T; ++v)
                if (load[v] < load[w]) w = v;
            load[w] += best_cost;
            o.mask[w] |= 1u << best;
        }
        return o;
    }
    static constexpr unsigned own(int w) { return owners().mask[w]; }

    // harmonic m-columns of each wavefront: contiguous ranges minimising the
    // slowest wavefront's VALU count.  Column m costs one instruction for
    // degree m + 1 and three per further degree plus one store per degree;
    // reaching T_m by the Chebyshev ladder costs two per step past m = 1.
    struct Split {
        int lo[4], hi[4];
    };
    static constexpr int column_cost(int m) {
        return (m < LM ? 1 : 0) + 3 * (LM - m - 1 > 0 ? LM - m - 1 : 0) + (LM - m + 1);
    }
    static constexpr int range_cost(int a, int b) {
        if (a >= b) return 0;
        int c = 2 * (b - 1 > 1 ? b - 2 : 0);
        for (int m = a; m < b; ++m) c += column_cost(m);
        return c;
    }
    static constexpr Split split() {
        constexpr int kInf = 1 << 29;
        int best[5][L + 1] = {};
        int cut[5][L + 1] = {};
        for (int w = 0; w <= T; ++w)
            for (int i = 0; i <= L; ++i) best[w][i] = kInf;
        best[0][0] = 0;
        for (int w = 1; w <= HW; ++w) {
            for (int i = 0; i <= L; ++i) {
                for (int j = 0; j <= i; ++j) {
                    if (best[w - 1][j] == kInf) continue;
                    const int c = best[w - 1][j] > range_cost(j, i) ? best[w - 1][j] : range_cost(j, i);
                    if (c < best[w][i]) {
                        best[w][i] = c;
                        cut[w][i] = j;
                    }
                }
            }
        }
        Split s{};
        int i = L;
        for (int w = HW; w >= 1; --w) {
            const int j = cut[w][i];
            s.lo[w - 1] = j;
            s.hi[w - 1] = i;
            i = j;
        }
        return s;
    }
    static constexpr int mlo(int w) { return split().lo[w]; }
    static constexpr int mhi(int w) { return split().hi[w]; }
};

// owned (l, cg) pairs before degree l, and in total, for a wavefront's mask
constexpr int units_before(unsigned mask, int l) {
    int u = 0;
    for (int i = 0; i < l; ++i)
        if ((mask >> i) & 1u) u += cgroups(i);
    return u;
}
constexpr int units_total(unsigned mask, int L) { return units_before(mask, L); }
constexpr int degrees_before(unsigned mask, int l) {
    int d = 0;
    for (int i = 0; i < l; ++i)
        if ((mask >> i) & 1u) ++d;
    return d;
}
constexpr int popcount_c(unsigned m) { return m == 0 ? 0 : (int)(m & 1u) + popcount_c(m >> 1); }

template <typename F, int... Is>
__device__ __forceinline__ void static_for(F&& f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void unroll(F&& f) {
    static_for(f, std::make_integer_sequence<int, N>{});
}

// --------------------------------------------------------------- device ---

__device__ __forceinline__ double mfma4(double a, double b, double c) {
    return __builtin_amdgcn_mfma_f64_4x4x4f64(a, b, c, 0, 0, 0);
}

// value of lane (L - k) mod 16 within each 16-lane row (DPP row rotate right
// by k lanes): block b takes block (b - k / 4) mod 4
template <int kLanes>
__device__ __forceinline__ double row_rotate(double v) {
    constexpr int ctrl = 0x120 + kLanes; // row_ror:kLanes (every lane reads a lane of its own row)
    const int lo = __builtin_amdgcn_mov_dpp(__double2loint(v), ctrl, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_mov_dpp(__double2hiint(v), ctrl, 0xF, 0xF, false);
    return __hiloint2double(hi, lo);
}

// value of lane L ^ 4 (block b takes block b ^ 1, columns unchanged)
__device__ __forceinline__ double swap_blocks(double v) {
    constexpr int pattern = 0x1F | (4 << 10); // swizzle bit mode: and 0x1f, or 0, xor 4
    const int lo = __builtin_amdgcn_ds_swizzle(__double2loint(v), pattern);
    const int hi = __builtin_amdgcn_ds_swizzle(__double2hiint(v), pattern);
    return __hiloint2double(hi, lo);
}

// exp(x) for x = -a d2 (a >= 0, d2 >= 0, x >= -708) by Tang's table method
// (ACM TOMS 15(2), 1989) with 256 entries: x = (256k + j) ln2/256 + r,
// |r| <= ln2/512, exp(x) = 2^k 2^(j/256) e^r with e^r - 1 by a short
// Taylor polynomial (below).  tab[j] = 2^(j/256)
// with j << 12 taken off its high word, so that adding (256k + j) << 12
// scales it by 2^k in one integer add (the result is a normal number for
// x >= -708).
//   kScaled false (float64 rows): na = -a, degree 4 (truncation below 4e-17
// relative).  x is rounded exactly as the
// reference's exp(-a * d2) argument (soap.cpp:895-896); the reduction is one
// fma against ln2/256 rounded to a double (relative error 3.4e-17), which
// puts |x| * 3.4e-17 of relative error on the result: less than the rounding
// of x itself (|x| * 1.1e-16) that the reference's own argument carries.
//   kScaled true (float32 rows): na = -a 256/ln2, rounded once on the host,
// so y = x 256/ln2 comes from one fma with the shifter and the reduced
// argument r = y - (256k + j) from a second (no product of its own), and
// e^r by its degree-3 Taylor polynomial (truncation below 1.4e-13 relative)
// evaluated as 1 + (e^r - 1) and scaled by the table entry in one multiply:
// two instructions fewer per exp, for |x| * 2.2e-16 + 1.4e-13 of relative
// error against the reference's exp -- far under the float32 rows' 2e-5 gate
// even after the beta fold's cancellation (2.3e5-fold for 8 channels: 3e-8).
template <bool kScaled>
__device__ __forceinline__ double exp_neg(double d2, double na, const int2* tab) {
    constexpr double kInvLn2xT = 369.32993046757463228414071833648; // 256 / ln 2
    constexpr double kLn2OverT = 0.0027076061740622863;              // ln 2 / 256
    constexpr double kShifter = 6755399441055744.0;                  // 1.5 * 2^52
    double s, r, q;
    if constexpr (kScaled) {
        s = fma(na, d2, kShifter);
        const double kf = s - kShifter;
        r = fma(na, d2, -kf); // in units of ln2/256, |r| <= 1/2
        // e^(c r) - 1 = r (c + r (c^2/2 + r (c^3/6 + r c^4/24))), c = ln2/256
        // e^(c r) = 1 + r (c + r (c^2/2 + r c^3/6)), c = ln2/256
        constexpr double c = kLn2OverT;
        q = fma(r, c * c * c / 6.0, c * c / 2.0);
        q = fma(q, r, c);
        q = fma(q, r, 1.0);
    } else {
        const double x = na * d2;
        s = fma(x, kInvLn2xT, kShifter);
        const double kf = s - kShifter;
        r = fma(kf, -kLn2OverT, x);
        q = fma(r, 1.0 / 24.0, 1.0 / 6.0);
        q = fma(q, r, 0.5);
        q = fma(q, r, 1.0);
    }
    const int nj = __double2loint(s);
    const int2 t = *reinterpret_cast<const int2*>(reinterpret_cast<const char*>(tab) +
                                                  ((nj << 3) & ((kTab - 1) << 3)));
    const double tk = __hiloint2double(t.y + (nj << (20 - kTabBits)), t.x); // 2^k 2^(j/256)
    if constexpr (kScaled) return tk * q;
    const double em1 = r * q; // e^r - 1
    return fma(tk, em1, tk);
}

// the lane constant of exp_neg<kScaled> for the exponent a
inline double exp_lane_constant(double a, bool scaled) {
    return scaled ? -a * 369.32993046757463228414071833648 : -a;
}

// Column m of the scaled harmonics (harmonic_table.h) from T_m, one part per
// lane: comp 0 the cos part (entry l*l + l - m), comp 1 the sin part
// (l*l + l + m).  col0 is the lane's slot in the staging buffer.
template <int LM, int M>
__device__ __forceinline__ void harmonic_column(double tm, double z, double r2, int comp, double* col0) {
    double* col = col0 + (comp != 0 ? M : -M) * kYS;
    col[(M * M + M) * kYS] = tm;
    if constexpr (M < LM) {
        double q2 = tm;
        double q1 = z * tm;
        col[((M + 1) * (M + 1) + (M + 1)) * kYS] = q1;
        unroll<LM - M - 1>([&](auto i) {
            constexpr int l = M + 2 + decltype(i)::value;
            constexpr double c = kScaledHarmonic.c[l][M];
            const double q = fma(z, q1, -((c * r2) * q2));
            col[(l * l + l) * kYS] = q;
            q2 = q1;
            q1 = q;
        });
    }
}

// Columns [MLO, MHI) of one slot's scaled harmonics.  Both lanes of a slot run
// the Chebyshev ladder T_m = 2x T_{m-1} - (x^2+y^2) T_{m-2}, which gives the
// cos part Re (x+iy)^m from (T_0, T_1) = (s, s x) and the sin part Im (x+iy)^m
// from (0, s y); s is 1, or 0 for a pad slot.  The sin part of m = 0 is empty:
// those lanes skip that column.
template <int LM, int MLO, int MHI>
__device__ __forceinline__ void harmonic_columns(double x, double y, double z, double s, int comp, double* col0) {
    if constexpr (MLO < MHI) {
        const double rho2 = fma(x, x, y * y);
        const double r2 = fma(z, z, rho2);
        const double tx = x + x;
        double t0 = comp != 0 ? 0.0 : s;
        double t1 = (comp != 0 ? y : x) * s;
        unroll<MHI>([&](auto mc) {
            constexpr int m = decltype(mc)::value;
            double tm;
            if constexpr (m == 0) {
                tm = t0;
            } else if constexpr (m == 1) {
                tm = t1;
            } else {
                tm = fma(tx, t1, -(rho2 * t0));
                t0 = t1;
                t1 = tm;
            }
            if constexpr (m >= MLO) {
                if constexpr (m == 0) {
                    if (comp == 0) harmonic_column<LM, 0>(tm, z, r2, comp, col0);
                } else {
                    harmonic_column<LM, m>(tm, z, r2, comp, col0);
                }
            }
        });
    }
}

// a wave-uniform 64-bit value in scalar registers
__device__ __forceinline__ int64_t uniform64(int64_t v) {
    const int lo = __builtin_amdgcn_readfirstlane(static_cast<int>(v));
    const int hi = __builtin_amdgcn_readfirstlane(static_cast<int>(v >> 32));
    return static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo));
}

template <int LM, int KG, int NCR, int ES, int MODE, int W>
__device__ __forceinline__ void block_role(const BlockArgs& a, double* lds, const int* s_ps, double* s_acc) {
    using PL = BlockPlan<LM, KG>;
    constexpr int L = PL::L, R = PL::R, P = PL::P, RPL = PL::RPL, NT = PL::NT, GS = PL::GS;
    constexpr int GROUPS = PL::GROUPS;
    constexpr unsigned kOwn = PL::own(W);
    constexpr int NU = units_total(kOwn, L); // owned (l, cg) pairs
    constexpr int ND = popcount_c(kOwn);     // owned degrees
    constexpr int MLO = PL::mlo(W), MHI = PL::mhi(W);
    constexpr bool kHarm = W < PL::HW; // this role stages harmonics (and loads the slots' positions)

    const int lane = threadIdx.x % kWaveThreads;
    const int S = a.S;
    double* s_y = lds;                                        // 2 x YWORDS
    double* s_d2 = s_y + 2 * PL::YWORDS;                      // 2 x kNb
    const int2* s_tab = reinterpret_cast<const int2*>(s_d2 + 2 * kNb); // kTab
    const double* s_scale = s_d2 + 2 * kNb + kTab;           // padded S_lm table

    // lane constants of the owned degrees
    double e1[ND > 0 ? ND : 1][RPL];
    double bt[ND > 0 ? ND : 1][NT];
    unroll<L>([&](auto lc) {
        constexpr int l = decltype(lc)::value;
        if constexpr ((kOwn >> l) & 1u) {
            constexpr int d = degrees_before(kOwn, l);
            unroll<RPL>([&](auto rc) {
                constexpr int rr = decltype(rc)::value;
                e1[d][rr] = a.lane_e1[(l * RPL + rr) * kWaveThreads + lane];
            });
            unroll<NT>([&](auto tc) {
                constexpr int t = decltype(tc)::value;
                bt[d][t] = a.lane_beta[(l * NT + t) * kWaveThreads + lane];
            });
        }
    });
    const int blk = (lane / 4) % 4;
    const int ph = blk / R;
    // staging reads: B operand of (l, cg) at (l*l + 4 cg) kYS + GS g + yread,
    // the lane's slot's d2 of step group g at GS g + dread.  A 64-bit LDS
    // read is served 16 lanes at a time; those lanes (one neighbour k) read 4
    // columns x P phases at a row pitch of 1 mod 16 doubles, all in
    // different banks.
    const int yread = (lane % 4) * kYS + 4 * ph + lane / 16;
    const int dread = 4 * ph + lane / 16;
    // lanes of the block slots {0, 1} (KG = 2: the even species' groups)
    const bool low_pair = (lane % 16) < 8;

    // ---------------------------------------------------------- slot stream
    // A centre's rows are grouped by species: cnt_t rows of species t after those of the species
    // before it.  The stream cuts each species' rows into chunks of at most 32
    // slots (a chunk never mixes species; its last step group may hold pad
    // slots past the rows) and runs two chunks ahead of the contraction: each
    // lane pair (two lanes per slot) loads the bin of its slot's row.  All of
    // its state but the loaded bins is wave-uniform.
    // Work: items [first, last) of this workgroup -- centres, or with
    // structure averages whole structures, whose centres are consecutive
    const int64_t work_first = a.item_base + static_cast<int64_t>(blockIdx.x) * a.per_block;
    const int64_t work_last = min(work_first + a.per_block, a.item_base + a.items);
    // rows of structure averages (the runs' launch sums a run of a structure's
    // centres the same way, into a partial row)
    constexpr bool inner = MODE == kBlockInner || MODE == kBlockInnerSmall || MODE == kBlockInnerRuns ||
                           MODE == kBlockInnerRunsWeighted || MODE == kBlockOuterLds;
    // outer averages in LDS: a structure's centres one by one, each centre's
    // power spectrum added into s_acc (F float64 values), its mean written
    // when the structure ends
    constexpr bool kOuter = MODE == kBlockOuterLds;
    constexpr bool kRuns = MODE == kBlockInnerRuns || MODE == kBlockInnerRunsWeighted;
    constexpr bool kFinal = MODE == kBlockInnerFinal;
    // this wavefront's registers in a partial row, and the row's width
    constexpr int kPartBase = [] {
        int u = 0;
        for (int w = 0; w < W; ++w) u += units_total(PL::own(w), L);
        return u;
    }() * NCR * kWaveThreads;
    constexpr int64_t kPartWidth = static_cast<int64_t>(units_total(0xffffffffu, L)) * NCR * kWaveThreads;
    // neighbour weights scale the harmonic seeds
    constexpr bool kWeighted = MODE == kBlockRowsWeighted || MODE == kBlockInnerRunsWeighted;
    constexpr bool kSummed = MODE == kBlockRowsSummed;     // mu1nu1: against the species-summed coefficients
    // structures of at most a wavefront of atoms: pairs streamed species-major
    // across the structure's centres (an average sums them in any order)
    constexpr bool kSpeciesMajor = MODE == kBlockInnerSmall;
    const int64_t item_first = inner ? uniform64(a.struct_offsets[work_first]) : work_first;
    const int64_t item_last = inner ? uniform64(a.struct_offsets[work_last]) : work_last;
    // structure of the stream's centre and its centre range (inner)
    int64_t st_struct = work_first - 1, st_struct_end = item_first;
    int pre_count = 0;     // next centre: rows of species t at lane t
    int64_t pre_start = 0; // next centre: first pair row (lane 0)
    // Loads are unconditional in every lane (clamped to valid addresses) so
    // that no merge of a loaded value forces an early wait for it.
    auto prefetch_centre = [&](int64_t c) {
        if (c < item_last) {
            // the lane (species) index is recomputed here rather than kept
            // live across the whole loop
            int t;
            asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(t));
            t = min(t, S - 1);
            pre_count = a.counts[c * S + t];
            pre_start = a.pair_start[c];
        }
    };
    int cnt = 0;                       // stream centre: rows of species t at lane t
    int64_t st_centre = item_first - 1;
    int64_t st_row = 0;                // pair row of the next chunk's first slot
    int st_q = 0;                      // species of the next chunk
    int st_left = 0;                   // rows of species st_q not yet in a chunk
    uint32_t st_more = 0;              // species after st_q with rows (bit mask)
    auto next_species = [&]() {
        st_q = __builtin_amdgcn_readfirstlane(__builtin_ctz(st_more));
        st_more = __builtin_amdgcn_readfirstlane(st_more & (st_more - 1));
        st_left = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(cnt, st_q));
    };
    auto enter_centre = [&]() {
        st_centre = uniform64(st_centre + 1);
        if constexpr (inner) {
            // skip to the centre's structure (empty structures have no centres)
            while (st_centre >= st_struct_end) {
                st_struct = uniform64(st_struct + 1);
                st_struct_end = uniform64(a.struct_offsets[st_struct + 1]);
            }
        }
        cnt = pre_count;
        st_row = uniform64(pre_start);
        st_more = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(__ballot(lane < S && cnt > 0)));
        cnt = lane < S ? cnt : 0;
        prefetch_centre(st_centre + 1);
        st_left = 0;
        if (st_more != 0) next_species();
    };
    // Species-major stream (structures of at most 64 atoms): lane i stands
    // for centre i of the structure.  For species q the structure's rows of
    // that species, centre after centre, form one sequence cut into chunks;
    // a slot finds its centre by a binary search over the centres' running
    // row totals (end_i) and its row at rowbase_i + (slot - first slot of
    // centre i), rowbase_i being the centre's first row of species q.
    int64_t sm_a0 = 0;      // first atom (centre) of the structure
    int sm_n = 0;           // its atoms
    int sm_total = 0;       // rows of species st_q over the structure
    int sm_base = 0;        // first slot of the next chunk
    int64_t l_rowbase = 0;  // lane i: first row of species st_q of centre i
    int l_cnt = 0;          // lane i: rows of species st_q of centre i
    int l_end = 0;          // lane i: rows of species st_q of centres 0..i
    auto sm_species = [&]() {
        st_q = __builtin_amdgcn_readfirstlane(__builtin_ctz(st_more));
        st_more = __builtin_amdgcn_readfirstlane(st_more & (st_more - 1));
        // the rows of the species before (none between: they have no rows)
        l_rowbase += l_cnt;
        l_cnt = lane < sm_n ? a.counts[(sm_a0 + lane) * S + st_q] : 0;
        int v = l_cnt;
#pragma unroll
        for (int off = 1; off < kWaveThreads; off *= 2) {
            const int u = __shfl_up(v, off);
            if (lane >= off) v += u;
        }
        l_end = v;
        sm_total = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(v, kWaveThreads - 1));
        sm_base = 0;
    };
    auto sm_structure = [&]() -> bool {
        // the next structure with atoms, if any
        do {
            st_struct = uniform64(st_struct + 1);
        } while (st_struct < work_last &&
                 uniform64(a.struct_offsets[st_struct + 1]) == uniform64(a.struct_offsets[st_struct]));
        if (st_struct >= work_last) return false;
        sm_a0 = uniform64(a.struct_offsets[st_struct]);
        sm_n = __builtin_amdgcn_readfirstlane(static_cast<int>(uniform64(a.struct_offsets[st_struct + 1]) - sm_a0));
        l_rowbase = lane < sm_n ? a.pair_start[sm_a0 + lane] : 0;
        l_cnt = 0;
        // species with rows in the structure
        uint32_t present = 0;
        for (int t = 0; t < S; ++t) {
            const int c = lane < sm_n ? a.counts[(sm_a0 + lane) * S + t] : 0;
            if (__ballot(c > 0) != 0) present |= 1u << t;
        }
        st_more = __builtin_amdgcn_readfirstlane(present);
        return true;
    };
    // pipeline stage of one chunk; everything but the bin and the centre is
    // wave-uniform
    struct Stage {
        int64_t centre; // -1: no chunk (species-major: the structure)
        int q;          // species
        int rows;       // rows in the chunk (slots past them are pad slots)
        int groups;     // step groups
        bool ends;      // last chunk of its centre
        bool last;      // last chunk of its output row: of its centre, or of its structure (inner)
        uint32_t bin;   // bin of the lane's slot row (slot < rows)
        int64_t row;    // output row (centre, or structure)
        int catom;      // species-major: centre (atom) of the lane's slot
        double w;       // weighted modes: weight of the lane's slot row
    };
    auto next_stage = [&]() -> Stage {
        Stage s{-1, 0, 0, 0, false, false, 0u, 0, 0, 0.0};
        if constexpr (kSpeciesMajor) {
            if (sm_base >= sm_total) {
                if (st_more == 0) {
                    if (!sm_structure()) return s;
                    if (st_more == 0) {
                        // no rows at all: an empty chunk ends the structure (a zero row)
                        s.centre = st_struct;
                        s.q = st_q;
                        s.ends = s.last = true;
                        s.row = st_struct;
                        return s;
                    }
                }
                sm_species();
            }
            const int n = min(sm_total - sm_base, kNb);
            s.centre = st_struct;
            s.q = st_q;
            s.rows = n;
            s.groups = (n + GS - 1) / GS;
            if constexpr (kHarm) {
                // pad slots repeat the chunk's last slot
                const int slot = sm_base + min(lane / 2, n - 1);
                // centre of the slot: the first whose running total exceeds it
                int lo = 0, hi = sm_n - 1;
#pragma unroll
                for (int it = 0; it < 6; ++it) {
                    const int mid = (lo + hi) / 2;
                    const bool right = __shfl(l_end, mid) <= slot;
                    lo = right ? mid + 1 : lo;
                    hi = right ? hi : mid;
                }
                const int before = __shfl(l_end, lo) - __shfl(l_cnt, lo);
                const int64_t base = static_cast<int64_t>(
                    (static_cast<uint64_t>(static_cast<uint32_t>(__shfl(static_cast<int>(l_rowbase >> 32), lo))) << 32) |
                    static_cast<uint32_t>(__shfl(static_cast<int>(l_rowbase), lo)));
                s.bin = a.pair_bin[base + (slot - before)];
                s.catom = static_cast<int>(sm_a0) + lo;
            }
            sm_base = __builtin_amdgcn_readfirstlane(sm_base + n);
            s.last = sm_base >= sm_total && st_more == 0;
            s.ends = s.last;
            s.row = st_struct;
            return s;
        }
        if (st_left == 0) {
            if (st_more != 0) {
                next_species();
            } else {
                if (st_centre + 1 >= item_last) return s;
                enter_centre();
            }
        }
        const int n = min(st_left, kNb);
        s.centre = st_centre;
        s.q = st_q;
        s.rows = n;
        s.groups = (n + GS - 1) / GS;
        // pad slots load the chunk's last row (a centre always has its own
        // row, so row 0 of the graph exists for an empty chunk)
        if constexpr (kHarm) {
            const int64_t slot_row = n > 0 ? st_row + min(lane / 2, n - 1) : 0;
            s.bin = a.pair_bin[slot_row];
            if constexpr (kWeighted) s.w = a.row_w[slot_row];
        }
        st_row = uniform64(st_row + n);
        st_left = __builtin_amdgcn_readfirstlane(st_left - n);
        s.ends = st_left == 0 && st_more == 0;
        s.last = s.ends;
        s.row = st_centre;
        if constexpr (inner) {
            // the structure's average: one row when its last centre ends
            s.last = s.ends && st_centre + 1 == st_struct_end;
            s.row = st_struct;
        }
        return s;
    };

    // accumulators and coefficient registers
    double acc[NU > 0 ? NU : 1][RPL];
    double C[NU > 0 ? NU : 1][NCR];
    unroll<NU>([&](auto u) {
        unroll<RPL>([&](auto r) { acc[decltype(u)::value][decltype(r)::value] = 0.0; });
        unroll<NCR>([&](auto r) { C[decltype(u)::value][decltype(r)::value] = 0.0; });
    });
    int cur = -1; // species of the accumulators

    // sum the phases of every accumulator and add species q's radial groups
    // into its block slots of the coefficient registers, which start every
    // output row at zero (a species merges once per centre; a structure
    // average adds its centres' sums): per lane and register a factor of 1
    // (the lane's block slot and the register belong to q) or 0, and one fma
    // per register
    auto merge = [&](int q_in) {
        // mu2: one coefficient species, the first species' slots
        const int q = a.mu2 != 0 ? 0 : q_in;
        const int rt = KG == 2 ? q >> 1 : KG == 1 ? q >> 2 : q;
        double sel[RPL][NCR];
        unroll<RPL>([&](auto rc) {
            constexpr int rr = decltype(rc)::value;
            bool mine;
            if constexpr (KG == 2) {
                mine = low_pair == ((q & 1) == 0);
            } else if constexpr (KG == 1) {
                mine = blk == (q & 3);
            } else {
                mine = blk == rr;
            }
            unroll<NCR>([&](auto r) { sel[rr][decltype(r)::value] = mine && rt == decltype(r)::value ? 1.0 : 0.0; });
        });
        unroll<NU>([&](auto uc) {
            constexpr int u = decltype(uc)::value;
            unroll<RPL>([&](auto rc) {
                constexpr int rr = decltype(rc)::value;
                double v = acc[u][rr];
                v += row_rotate<8>(v);
                if constexpr (P == 4) v += row_rotate<4>(v);
                acc[u][rr] = 0.0;
                unroll<NCR>([&](auto r) {
                    constexpr int ri = decltype(r)::value;
                    C[u][ri] = fma(v, sel[rr][ri], C[u][ri]);
                });
                __builtin_amdgcn_sched_barrier(0);
            });
        });
    };

    const int64_t F = a.F;
    // row end: C <- (S_lm C)^T beta^T scaled by scale0, the power spectrum of
    // the owned degrees to output row row0, and C back to zero
    auto row_end = [&](int64_t row0, double scale0) {
        // fold: C <- (S_lm C)^T beta^T in place
        unroll<L>([&](auto lc) {
            constexpr int l = decltype(lc)::value;
            if constexpr ((kOwn >> l) & 1u) {
                constexpr int d = degrees_before(kOwn, l);
                constexpr int u0 = units_before(kOwn, l);
                constexpr int loff = 4 * units_before(0xffffffffu, l);
                unroll<cgroups(l)>([&](auto cc) {
                    constexpr int cg = decltype(cc)::value;
                    const double sc = s_scale[loff + 4 * cg + lane % 4] * scale0;
                    unroll<NCR>([&](auto rc) {
                        constexpr int r = decltype(rc)::value;
                        const double v = C[u0 + cg][r] * sc;
                        double c = mfma4(v, bt[d][0], 0.0);
                        if constexpr (KG == 2) {
                            c = mfma4(swap_blocks(v), bt[d][1], c);
                        } else if constexpr (KG == 3) {
                            c = mfma4(row_rotate<12>(v), bt[d][1], c); // block b takes b + 1
                            c = mfma4(row_rotate<8>(v), bt[d][2], c);  // b + 2
                            c = mfma4(row_rotate<4>(v), bt[d][3], c);  // b + 3
                        }
                        C[u0 + cg][r] = c;
                        __builtin_amdgcn_sched_barrier(0);
                    });
                });
            }
        });
        // power spectrum of the owned degrees, written to the centre's row
        char* row = static_cast<char*>(a.out) + row0 * a.pitch;
        const __amdgpu_buffer_rsrc_t rsrc =
            __builtin_amdgcn_make_buffer_rsrc(row, 0, static_cast<int>(F * ES), 0x00020000);
        // one 4-value store per lane and value of a Gram tile (outer
        // averages: added into the structure's row in LDS, each feature by
        // one lane; the pairs not stored are past the row)
        auto store_tile = [&](const d4& D, const int* fb, const int* fs, int l) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const double v = D[r]; // the coefficients carry sqrt(pi sqrt(8/(2l+1)))
                const int off = fb[r] + l * fs[r];
                if constexpr (kOuter) {
                    if (off < static_cast<int>(F * ES)) s_acc[off / ES] += v;
                } else if constexpr (ES == 4) {
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(static_cast<float>(v)), rsrc, off, 0, 0);
                } else {
                    typedef int i2v __attribute__((ext_vector_type(2)));
                    const i2v bits = {__double2loint(v), __double2hiint(v)};
                    __builtin_amdgcn_raw_buffer_store_b64(bits, rsrc, off, 0, 0);
                }
            }
        };
        if constexpr (kSummed) {
            // species-summed coefficients: the registers added, then the
            // species' blocks of a register (KG 2: b and b ^ 2; KG 1: all
            // four; KG 3 holds one species)
            double cs[NU > 0 ? NU : 1];
            unroll<NU>([&](auto uc) {
                constexpr int u = decltype(uc)::value;
                double v = C[u][0];
                unroll<NCR - 1>([&](auto rc) { v += C[u][decltype(rc)::value + 1]; });
                if constexpr (KG == 2) {
                    v += row_rotate<8>(v);
                } else if constexpr (KG == 1) {
                    v += row_rotate<8>(v);
                    v += row_rotate<4>(v);
                }
                cs[u] = v;
            });
            unroll<NCR>([&](auto ic) {
                constexpr int ri = decltype(ic)::value;
                int fb[4], fs[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int o = s_ps[(ri * 4 + r) * kWaveThreads + lane];
                    fb[r] = o >> kStrideBits; // bytes
                    fs[r] = (o & ((1 << kStrideBits) - 1)) * ES;
                }
                unroll<L>([&](auto lc) {
                    constexpr int l = decltype(lc)::value;
                    if constexpr ((kOwn >> l) & 1u) {
                        constexpr int u0 = units_before(kOwn, l);
                        d4 D = {0.0, 0.0, 0.0, 0.0};
                        unroll<cgroups(l)>([&](auto cc) {
                            constexpr int cg = decltype(cc)::value;
                            D = mfma(C[u0 + cg][ri], cs[u0 + cg], D);
                        });
                        store_tile(D, fb, fs, l);
                    }
                });
            });
        }
        int pair = 0;
        unroll<NCR>([&](auto ic) {
            constexpr int ri = decltype(ic)::value;
            unroll<NCR>([&](auto jc) {
                constexpr int rj = decltype(jc)::value;
                if constexpr (!kSummed && ri <= rj) {
                    int fb[4], fs[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int o = s_ps[(pair * 4 + r) * kWaveThreads + lane];
                        fb[r] = o >> kStrideBits; // bytes
                        fs[r] = (o & ((1 << kStrideBits) - 1)) * ES;
                    }
                    unroll<L>([&](auto lc) {
                        constexpr int l = decltype(lc)::value;
                        if constexpr ((kOwn >> l) & 1u) {
                            constexpr int u0 = units_before(kOwn, l);
                            d4 D = {0.0, 0.0, 0.0, 0.0};
                            unroll<cgroups(l)>([&](auto cc) {
                                constexpr int cg = decltype(cc)::value;
                                D = mfma(C[u0 + cg][ri], C[u0 + cg][rj], D);
                            });
                            store_tile(D, fb, fs, l);
                        }
                    });
                    ++pair;
                }
            });
        });
        unroll<NU>([&](auto u) { unroll<NCR>([&](auto r) { C[decltype(u)::value][decltype(r)::value] = 0.0; }); });
    };

    if constexpr (kFinal) {
        // structure rows from the sums of their partial rows (in order)
        for (int64_t s = work_first; s < work_last; ++s) {
            const int64_t r0 = uniform64(a.part_items[s]), r1 = uniform64(a.part_items[s + 1]);
            const double* part = a.partial_in + kPartBase + lane;
            unroll<NU>([&](auto uc) {
                unroll<NCR>([&](auto rc) {
                    constexpr int u = decltype(uc)::value, r = decltype(rc)::value;
                    double v = 0.0;
                    for (int64_t it = r0; it < r1; ++it) v += part[it * kPartWidth + (u * NCR + r) * kWaveThreads];
                    C[u][r] = v;
                });
            });
            const int64_t atoms = uniform64(a.struct_offsets[s + 1]) - uniform64(a.struct_offsets[s]);
            row_end(s, atoms > 0 ? 1.0 / static_cast<double>(atoms) : 0.0);
        }
        return;
    }

    if (!kSpeciesMajor && item_first < item_last) prefetch_centre(item_first);
    Stage s0 = next_stage(); // chunk k (contraction)
    Stage s1 = next_stage(); // chunk k + 1 (harmonics)
    double px = 0.0, py = 0.0, pz = 0.0;
    double qx = 0.0, qy = 0.0, qz = 0.0; // species-major: the slot's centre
    const int jj = lane / 2, comp = lane % 2;
    auto load_positions = [&](const Stage& s) {
        if constexpr (kHarm) {
            px = a.bx[s.bin];
            py = a.by[s.bin];
            pz = a.bz[s.bin];
            if constexpr (kSpeciesMajor) {
                qx = a.positions[3 * static_cast<int64_t>(s.catom)];
                qy = a.positions[3 * static_cast<int64_t>(s.catom) + 1];
                qz = a.positions[3 * static_cast<int64_t>(s.catom) + 2];
            }
        }
    };
    // harmonics of a stage's slots from the centre position (cx, cy, cz)
    auto harmonics = [&](const Stage& s, int buf, double cx, double cy, double cz) {
        const double dx = px - cx, dy = py - cy, dz = pz - cz;
        const bool real = jj < s.rows;
        if constexpr (W == 0) {
            // a pad slot's position is stale (a row of an earlier chunk,
            // possibly of another structure): it enters the exp as d2 = 0
            const double d2 = fma(dz, dz, fma(dx, dx, dy * dy));
            if (comp == 0) s_d2[buf * kNb + jj] = real ? d2 : 0.0;
        }
        double seed = real ? 1.0 : 0.0;
        // the neighbour's weight, computed per row before the expansion
        if constexpr (kWeighted) seed = real ? s.w : 0.0;
        harmonic_columns<LM, MLO, MHI>(dx, dy, dz, seed, comp, s_y + buf * PL::YWORDS + jj);
    };

    // prologue: harmonics of the first chunk
    load_positions(s0);
    if (kHarm && uniform64(s0.centre) >= 0) {
        if constexpr (kSpeciesMajor) {
            harmonics(s0, 0, qx, qy, qz);
        } else {
            const int64_t c = uniform64(s0.centre);
            harmonics(s0, 0, a.positions[3 * c], a.positions[3 * c + 1], a.positions[3 * c + 2]);
        }
    }
    load_positions(s1);
    __syncthreads();

    int k = 0;
    while (uniform64(s0.centre) >= 0) {
        const int buf = k & 1;
        // wave-uniform facts of chunk k, in scalar registers
        const int groups0 = __builtin_amdgcn_readfirstlane(s0.groups);
        const bool last0 = __builtin_amdgcn_readfirstlane(s0.last ? 1 : 0) != 0;
        const bool ends0 = inner ? __builtin_amdgcn_readfirstlane(s0.ends ? 1 : 0) != 0 : last0;
        const int64_t row0 = uniform64(s0.row);
        const int q0 = __builtin_amdgcn_readfirstlane(s0.q);
        // centre position of chunk k + 1 (scalar loads, used after the contraction)
        const int64_t centre1 = uniform64(s1.centre);
        const int64_t cpos1 = 3 * (centre1 >= 0 ? centre1 : 0);
        double cx1 = 0.0, cy1 = 0.0, cz1 = 0.0;
        if constexpr (kHarm && !kSpeciesMajor) {
            cx1 = a.positions[cpos1];
            cy1 = a.positions[cpos1 + 1];
            cz1 = a.positions[cpos1 + 2];
        }
        // positions of chunk k + 1 in flight; bins of chunk k + 2
        Stage s2 = next_stage();
        // ------------------------------------------------ contraction of chunk k
        {
            const int prev = __builtin_amdgcn_readfirstlane(cur);
            if (q0 != prev) {
                if (prev >= 0) merge(prev);
                cur = q0;
            }
            const double* ybuf = s_y + buf * PL::YWORDS + yread;
            const double* dbuf = s_d2 + buf * kNb + dread;
            unroll<GROUPS>([&](auto gc) {
                constexpr int g = decltype(gc)::value;
                if (g >= groups0) return;
                const double d2 = dbuf[GS * g];
                double ev[ND > 0 ? ND : 1][RPL];
                unroll<ND>([&](auto dc) {
                    unroll<RPL>([&](auto rc) {
                        ev[decltype(dc)::value][decltype(rc)::value] =
                            exp_neg<ES == 4>(d2, e1[decltype(dc)::value][decltype(rc)::value], s_tab);
                    });
                });
                unroll<L>([&](auto lc) {
                    constexpr int l = decltype(lc)::value;
                    if constexpr ((kOwn >> l) & 1u) {
                        constexpr int d = degrees_before(kOwn, l);
                        constexpr int u0 = units_before(kOwn, l);
                        unroll<cgroups(l)>([&](auto cc) {
                            constexpr int cg = decltype(cc)::value;
                            const double y = ybuf[(l * l + 4 * cg) * kYS + GS * g];
                            unroll<RPL>([&](auto rc) {
                                constexpr int rr = decltype(rc)::value;
                                acc[u0 + cg][rr] = mfma4(ev[d][rr], y, acc[u0 + cg][rr]);
                            });
                        });
                    }
                });
            });
        }
        // a centre's sums end in the coefficient registers (an average
        // thereby sums per-centre coefficients, as a centre's row does)
        if (ends0) {
            merge(__builtin_amdgcn_readfirstlane(cur));
            cur = -1;
            // outer averages: the centre's power spectrum into the row in LDS
            if constexpr (kOuter) row_end(row0, 1.0);
        }
        // ------------------------------------ row end: fold, power spectrum
        if (last0) {
            if constexpr (kOuter) {
                // every wavefront's additions are in: the mean to the
                // structure's row, the LDS row back to zero for the next
                __syncthreads();
                const double inv = 1.0 / static_cast<double>(uniform64(a.struct_offsets[row0 + 1]) -
                                                             uniform64(a.struct_offsets[row0]));
                char* orow = static_cast<char*>(a.out) + row0 * a.pitch;
                // (the plan's tables are those of float64 rows; the mean is
                // written in the output's type, a.outer_lds bytes)
                const bool f32 = a.outer_lds == 4;
                for (int64_t f = threadIdx.x; f < F; f += blockDim.x) {
                    const double v = s_acc[f] * inv;
                    s_acc[f] = 0.0;
                    if (f32) {
                        reinterpret_cast<float*>(orow)[f] = static_cast<float>(v);
                    } else {
                        reinterpret_cast<double*>(orow)[f] = v;
                    }
                }
                __syncthreads();
            } else if constexpr (kRuns) {
                // the run's summed coefficient registers to its partial row
                double* part = a.partial_out + row0 * kPartWidth + kPartBase + lane;
                unroll<NU>([&](auto uc) {
                    unroll<NCR>([&](auto rc) {
                        constexpr int u = decltype(uc)::value, r = decltype(rc)::value;
                        part[(u * NCR + r) * kWaveThreads] = C[u][r];
                        C[u][r] = 0.0;
                    });
                });
            } else {
                // an average's coefficients carry 1 / (atoms of the structure)
                double scale0 = 1.0;
                if constexpr (inner) {
                    scale0 = 1.0 / static_cast<double>(uniform64(a.struct_offsets[row0 + 1]) -
                                                       uniform64(a.struct_offsets[row0]));
                }
                row_end(row0, scale0);
            }
        }
        // ---------------------------------------- harmonics of chunk k + 1
        if (kHarm && centre1 >= 0) {
            if constexpr (kSpeciesMajor) {
                harmonics(s1, buf ^ 1, qx, qy, qz);
            } else {
                harmonics(s1, buf ^ 1, cx1, cy1, cz1);
            }
        }
        load_positions(s2);
        s0 = s1;
        s1 = s2;
        ++k;
        __syncthreads();
    }
}

// Gram tiles of the power-spectrum offset table: the register pairs ri <= rj,
// or (summed coefficients) the registers
constexpr int ps_tiles(int ncr, bool summed) { return summed ? ncr : ncr * (ncr + 1) / 2; }

// Five wavefronts per SIMD (96 VGPRs); four for mu1nu1, whose summed
// coefficients stay live beside the registers, and for outer averages in
// LDS (their row in LDS allows four workgroups a CU at most; with five the
// l_max 6 shape spills).  The weighted modes read each row's weight, so
// they keep five.
template <int LM, int KG, int NCR, int ES, int MODE>
__global__ __launch_bounds__(256) __attribute__((
    amdgpu_waves_per_eu(MODE == kBlockRowsSummed || MODE == kBlockOuterLds ? 4 : 5))) void
k_soap_block(BlockArgs a) {
    using PL = BlockPlan<LM, KG>;
    // staging buffers, d2, exp table, padded S_lm table, power-spectrum
    // offsets; sized at compile time, so every LDS offset is an immediate
    __shared__ double lds[2 * PL::YWORDS + 2 * kNb + kTab + 4 * units_before(0xffffffffu, PL::L)];
    // the plan's offset table: a tile per register pair, or (mu1nu1) one per
    // register against the species-summed one; no more is read
    constexpr int kPsWords = ps_tiles(NCR, MODE == kBlockRowsSummed) * 4 * kWaveThreads;
    __shared__ int s_ps[kPsWords];
    // outer averages in LDS: the structure's row (F float64), sized at launch
    extern __shared__ double s_acc[];
    const int tid = threadIdx.x;
    for (int i = tid; i < kPsWords; i += static_cast<int>(blockDim.x)) s_ps[i] = a.ps_offsets[i];
    const int threads = static_cast<int>(blockDim.x);
    double* s_y = lds;
    double* s_d2 = s_y + 2 * PL::YWORDS;
    int2* s_tab = reinterpret_cast<int2*>(s_d2 + 2 * kNb);
    double* s_scale = s_d2 + 2 * kNb + kTab;
    // the first rows of the second staging buffer, which the pad columns
    // of the first chunk read, start finite (zero); the exp table
    for (int i = tid; i < 3 * kYS; i += threads) s_y[PL::YWORDS + i] = 0.0;
    for (int i = tid; i < kTab; i += threads) {
        const double t = exp2(static_cast<double>(i) / kTab);
        s_tab[i] = int2{__double2loint(t), __double2hiint(t) - (i << (20 - kTabBits))};
    }
    {
        // S_lm of padded column i (degree l's block at 4 sum_{l' < l} cg(l'),
        // 4 cg(l) wide; 0 past 2l)
        constexpr int kPad = 4 * units_before(0xffffffffu, PL::L);
        for (int i = tid; i < kPad; i += threads) {
            int l = 0, off = 0;
            while (l + 1 < PL::L && off + 4 * cgroups(l) <= i) {
                off += 4 * cgroups(l);
                ++l;
            }
            const int c = i - off;
            // S_lm times the square root of the degree's power-spectrum
            // prefactor (the Gram product then carries the prefactor itself)
            s_scale[i] = c <= 2 * l ? kScaledHarmonic.s[l][c <= l ? l - c : c - l] * kPsRoot[l] : 0.0;
        }
    }
    if constexpr (MODE == kBlockOuterLds) {
        for (int64_t i = tid; i < a.F; i += threads) s_acc[i] = 0.0;
    }
    __syncthreads();
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWaveThreads);
    if (wave == 0) {
        block_role<LM, KG, NCR, ES, MODE, 0>(a, lds, s_ps, s_acc);
    } else if constexpr (PL::T > 1) {
        if (wave == 1) {
            block_role<LM, KG, NCR, ES, MODE, (PL::T > 1 ? 1 : 0)>(a, lds, s_ps, s_acc);
        } else if constexpr (PL::T > 2) {
            if (wave == 2) {
                block_role<LM, KG, NCR, ES, MODE, (PL::T > 2 ? 2 : 0)>(a, lds, s_ps, s_acc);
            } else if constexpr (PL::T > 3) {
                block_role<LM, KG, NCR, ES, MODE, (PL::T > 3 ? 3 : 0)>(a, lds, s_ps, s_acc);
            }
        }
    }
}

template <int LM, int KG, int NCR>
size_t lds_bytes() {
    using PL = BlockPlan<LM, KG>;
    return (2 * PL::YWORDS + 2 * kNb + kTab + 4 * units_before(0xffffffffu, PL::L)) * sizeof(double);
}

template <int LM, int KG, int NCR>
void launch_shape(hipStream_t stream, const BlockArgs& a, int64_t count) {
    using PL = BlockPlan<LM, KG>;
    // outer averages in LDS: the structure's float64 row beside the tables
    const size_t row_lds = a.outer_lds != 0 ? static_cast<size_t>(a.F) * sizeof(double) : 0;
    const size_t lds = lds_bytes<LM, KG, NCR>() + ps_tiles(NCR, a.summed != 0) * 4 * kWaveThreads * sizeof(int) +
                       row_lds;
    const int64_t resident = std::max<int64_t>(1, std::min<int64_t>(8, (160 * 1024) / std::max<size_t>(lds, 1)));
    const int64_t target = std::max<int64_t>(1, 8 * resident * device_compute_units());
    BlockArgs args = a;
    // atom-level rows: at least two centres a workgroup, so the exp table and
    // the stage pipeline are set up for more than one (config 1's expansion
    // 0.090 -> 0.085 ms); structure averages keep one structure a workgroup
    const int64_t least = a.struct_offsets != nullptr ? 1 : 2;
    args.per_block = std::max<int64_t>(least, (count + target - 1) / target);
    const unsigned grid = static_cast<unsigned>((count + args.per_block - 1) / args.per_block);
    const dim3 threads(PL::T * kWaveThreads);
    const int mode = a.outer_lds != 0            ? kBlockOuterLds
                     : a.partial_in != nullptr    ? kBlockInnerFinal
                     : a.partial_out != nullptr ? (a.species_w != nullptr ? kBlockInnerRunsWeighted : kBlockInnerRuns)
                     : a.struct_offsets != nullptr ? (a.small_structures ? kBlockInnerSmall : kBlockInner)
                     : a.species_w != nullptr ? kBlockRowsWeighted
                     : a.summed != 0          ? kBlockRowsSummed
                                              : kBlockRows;
    auto launch = [&](auto m) {
        constexpr int M = decltype(m)::value;
        const unsigned dyn = M == kBlockOuterLds ? static_cast<unsigned>(row_lds) : 0u;
        if (a.out_dtype == 4) {
            hipLaunchKernelGGL((k_soap_block<LM, KG, NCR, 4, M>), dim3(grid), threads, dyn, stream, args);
        } else {
            hipLaunchKernelGGL((k_soap_block<LM, KG, NCR, 8, M>), dim3(grid), threads, dyn, stream, args);
        }
    };
    if (mode == kBlockRows) {
        launch(std::integral_constant<int, kBlockRows>{});
    } else if (mode == kBlockInner) {
        launch(std::integral_constant<int, kBlockInner>{});
    } else if (mode == kBlockInnerSmall) {
        launch(std::integral_constant<int, kBlockInnerSmall>{});
    } else if (mode == kBlockRowsWeighted) {
        launch(std::integral_constant<int, kBlockRowsWeighted>{});
    } else if (mode == kBlockInnerRuns) {
        launch(std::integral_constant<int, kBlockInnerRuns>{});
    } else if (mode == kBlockInnerRunsWeighted) {
        launch(std::integral_constant<int, kBlockInnerRunsWeighted>{});
    } else if (mode == kBlockInnerFinal) {
        launch(std::integral_constant<int, kBlockInnerFinal>{});
    } else if (mode == kBlockOuterLds) {
        launch(std::integral_constant<int, kBlockOuterLds>{});
    } else {
        launch(std::integral_constant<int, kBlockRowsSummed>{});
    }
}

using Launcher = void (*)(hipStream_t, const BlockArgs&, int64_t);

// the shapes compiled: (l_max, radial groups, coefficient registers)
struct ShapeEntry {
    int l_max, kg, ncr;
    Launcher launch;
    int waves;
};
#define MDX_BLOCK_SHAPE(LM, KG, NCR) {LM, KG, NCR, &launch_shape<LM, KG, NCR>, BlockPlan<LM, KG>::T}
const ShapeEntry kShapes[] = {
    MDX_BLOCK_SHAPE(3, 1, 1), // water (benchmark configuration 1)
    MDX_BLOCK_SHAPE(6, 2, 2), // HCNO (configuration 2)
    MDX_BLOCK_SHAPE(4, 2, 3), // molecules (configuration 3)
    MDX_BLOCK_SHAPE(8, 2, 3), // high-entropy alloy (configuration 4)
    MDX_BLOCK_SHAPE(9, 3, 1), // liquid silicon (configuration 5)
};
#undef MDX_BLOCK_SHAPE

const ShapeEntry* find_shape(int l_max, int kg, int ncr) {
    for (const ShapeEntry& e : kShapes)
        if (e.l_max == l_max && e.kg == kg && e.ncr == ncr) return &e;
    return nullptr;
}

int coefficient_registers(int S, int kg) { return kg == 3 ? S : (S * kg + 3) / 4; }

} // namespace

int64_t block_partial_width(int l_max, int ncr) {
    return static_cast<int64_t>(units_total(0xffffffffu, l_max + 1)) * ncr * kWaveThreads;
}

bool block_plan_tables(int S, int n, int l_max, int out_dtype, int compression, const std::vector<double>& beta_scaled,
                       const std::vector<double>& pref, const std::vector<double>& expo, BlockPlanHost& out) {
    out = BlockPlanHost{};
    if (compression < 0 || compression > 3) return false;
    // species of the coefficients and the feature layout (mu2: one)
    const int St = compression == 1 ? 1 : S;
    const int kg = (n + 3) / 4;
    if (n < 1 || kg > 3 || (kg == 3 && S != 1)) return false;
    const int ncr = coefficient_registers(S, kg);
    const ShapeEntry* e = find_shape(l_max, kg, ncr);
    if (e == nullptr) return false;
    const int L = l_max + 1;
    {
        const int64_t W = static_cast<int64_t>(St) * n;
        const int64_t F = compression == 2 ? W * n * L : compression == 3 ? W * (n + 1) / 2 * L : W * (W + 1) / 2 * L;
        if (F * out_dtype >= kDroppedBytes || n * n >= (1 << kStrideBits)) return false;
    }
    const int R = kg == 2 ? 2 : 1;
    const int RPL = kg / R;
    const int NT = kg == 1 ? 1 : kg == 2 ? 2 : 4;
    auto beta = [&](int l, int np, int k) -> double {
        if (np >= n || k >= n || np < 0 || k < 0) return 0.0;
        return beta_scaled[static_cast<size_t>((l * n + np) * n + k)] * pref[static_cast<size_t>(l * n + k)];
    };
    out.lane_e1.assign(static_cast<size_t>(L) * RPL * 64, 0.0);
    out.lane_beta.assign(static_cast<size_t>(L) * NT * 64, 0.0);
    for (int l = 0; l < L; ++l) {
        for (int lane = 0; lane < 64; ++lane) {
            const int b = (lane / 4) % 4;
            for (int rr = 0; rr < RPL; ++rr) {
                const int rg = rr * R + b % R;
                const int k = 4 * rg + lane % 4;
                out.lane_e1[static_cast<size_t>((l * RPL + rr) * 64 + lane)] =
                    k < n ? exp_lane_constant(expo[static_cast<size_t>(l * n + k)], out_dtype == 4) : 0.0;
            }
            // beta^T operand: lane = beta^T[k = lane / 16][n' = lane % 4] of the
            // fold term's (radial group in -> radial group out) block
            for (int t = 0; t < NT; ++t) {
                double v = 0.0;
                if (kg == 1) {
                    v = beta(l, lane % 4, lane / 16);
                } else if (kg == 2) {
                    const int rg = b % 2;
                    const int rin = t == 0 ? rg : 1 - rg;
                    v = beta(l, 4 * rg + lane % 4, 4 * rin + lane / 16);
                } else {
                    const int rin = (b + t) % 4;
                    if (b < 3 && rin < 3) v = beta(l, 4 * b + lane % 4, 4 * rin + lane / 16);
                }
                out.lane_beta[static_cast<size_t>((l * NT + t) * 64 + lane)] = v;
            }
        }
    }
    // power-spectrum offsets: tile pair p = (ri <= rj), value r, lane: feature
    // index at l = 0 and its stride per degree for channel i (group 4 ri + r,
    // radial channel 4 rg + lane / 16) and channel j (group 4 rj + (lane % 16) / 4,
    // 4 rg + lane % 4); pairs i > j and pad channels get kDroppedBytes
    auto channel = [&](int ri, int slot, int nl) -> int {
        int t = 0, rg = 0;
        if (kg == 3) {
            t = ri;
            rg = slot;
            if (slot >= 3) return -1;
        } else {
            const int g = 4 * ri + slot;
            t = g / kg;
            rg = g % kg;
        }
        const int np = 4 * rg + nl;
        if (t >= St || np >= n) return -1;
        return t * n + np;
    };
    // feature index of channel pair (i, j), i <= j (soap.cpp:997-1013)
    auto feature = [&](int i, int j, int& stride) -> int {
        const int t1 = i / n, n1 = i % n, t2 = j / n, n2 = j % n;
        int base = 0;
        for (int a1 = 0; a1 < St; ++a1) {
            for (int a2 = a1; a2 < St; ++a2) {
                const int size = a1 == a2 ? n * (n + 1) / 2 : n * n;
                if (a1 == t1 && a2 == t2) {
                    stride = size;
                    return base + (t1 == t2 ? n1 * n - n1 * (n1 - 1) / 2 + (n2 - n1) : n1 * n + n2);
                }
                base += L * size;
            }
        }
        return -1;
    };
    if (compression == 2) {
        // mu1nu1 (soap.cpp:969-981): channel i = (t, n1) of register ri
        // against the species-summed channel n2, feature t L n^2 + l n^2 +
        // n1 n + n2.  The summed register repeats its channels in every
        // species' blocks; its first kg blocks are taken.
        for (int ri = 0; ri < ncr; ++ri) {
            for (int r = 0; r < 4; ++r) {
                for (int lane = 0; lane < 64; ++lane) {
                    const int i = channel(ri, r, lane / 16);
                    const int slot = (lane % 16) / 4;
                    const int j = slot < kg ? 4 * slot + lane % 4 : n;
                    int fb = kDroppedBytes, fs = 0;
                    if (i >= 0 && j < n) {
                        const int t = i / n;
                        fb = (t * L * n * n + (i - t * n) * n + j) * out_dtype;
                        fs = n * n;
                    }
                    out.ps_offsets.push_back((fb << kStrideBits) | fs);
                }
            }
        }
    } else {
        for (int ri = 0; ri < ncr; ++ri) {
            for (int rj = ri; rj < ncr; ++rj) {
                for (int r = 0; r < 4; ++r) {
                    for (int lane = 0; lane < 64; ++lane) {
                        const int i = channel(ri, r, lane / 16);
                        const int j = channel(rj, (lane % 16) / 4, lane % 4);
                        int fb = kDroppedBytes, fs = 0;
                        if (i >= 0 && j >= 0 && i <= j) {
                            if (compression == 3) {
                                // crossover (soap.cpp:983-995): same species only
                                const int t1 = i / n, t2 = j / n, n1 = i % n, n2 = j % n;
                                if (t1 == t2) {
                                    fs = n * (n + 1) / 2;
                                    fb = (t1 * L * fs + n1 * n - n1 * (n1 - 1) / 2 + (n2 - n1)) * out_dtype;
                                }
                            } else {
                                fb = feature(i, j, fs) * out_dtype;
                            }
                        }
                        out.ps_offsets.push_back((fb << kStrideBits) | fs);
                    }
                }
            }
        }
    }
    // the kernel stages exactly this many entries
    if (out.ps_offsets.size() != static_cast<size_t>(ps_tiles(ncr, compression == 2)) * 4 * 64) {
        throw Error(MDX_INTERNAL, "power-spectrum offset table does not match the expansion kernel");
    }
    out.kg = kg;
    out.ncr = ncr;
    out.waves = e->waves;
    return true;
}


void launch_block_expand(hipStream_t stream, int l_max, int kg, int ncr, const BlockArgs& a, int64_t count) {
    if (count <= 0) return;
    const ShapeEntry* e = find_shape(l_max, kg, ncr);
    if (e == nullptr) throw Error(MDX_INTERNAL, "SOAP shape is not compiled for the register-coefficient kernel");
    if (a.outer_lds != 0 && (a.struct_offsets == nullptr || a.out_dtype != 8 ||
                             a.F * static_cast<int64_t>(sizeof(double)) > kBlockOuterLdsBytes)) {
        throw Error(MDX_INTERNAL, "outer average row does not fit the register-coefficient kernel's LDS");
    }
    e->launch(stream, a, count);
    MDX_HIP(hipGetLastError());
}

namespace {

// a wavefront per centre, kRowsPerLane of its rows per lane at a time: every
// row's loads are issued before any weight is formed, so the gathers of
// the batch of rows are in flight together; the distance as the
// expansion's harmonic staging forms it (image - centre, fma order)
constexpr int kRowsPerLane = 4;
__global__ __launch_bounds__(256) void k_block_row_weights(BlockArgs a, int64_t centres, double* row_w) {
    const int lane = threadIdx.x % kWaveThreads;
    const int64_t waves = static_cast<int64_t>(gridDim.x) * (blockDim.x / kWaveThreads);
    for (int64_t c = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWaveThreads) + threadIdx.x / kWaveThreads;
         c < centres; c += waves) {
        int total = 0;
        for (int t = 0; t < a.S; ++t) total += a.counts[c * a.S + t];
        const int64_t row0 = a.pair_start[c];
        const double cx = a.positions[3 * c], cy = a.positions[3 * c + 1], cz = a.positions[3 * c + 2];
        for (int base = 0; base < total; base += kRowsPerLane * kWaveThreads) {
            uint32_t bin[kRowsPerLane];
            double px[kRowsPerLane], py[kRowsPerLane], pz[kRowsPerLane];
#pragma unroll
            for (int i = 0; i < kRowsPerLane; ++i) {
                const int r = base + i * kWaveThreads + lane;
                bin[i] = r < total ? a.pair_bin[row0 + r] : a.pair_bin[row0];
            }
#pragma unroll
            for (int i = 0; i < kRowsPerLane; ++i) {
                px[i] = a.bx[bin[i]];
                py[i] = a.by[bin[i]];
                pz[i] = a.bz[bin[i]];
            }
#pragma unroll
            for (int i = 0; i < kRowsPerLane; ++i) {
                const int r = base + i * kWaveThreads + lane;
                if (r >= total) continue;
                const uint32_t b = bin[i];
                const double dx = px[i] - cx, dy = py[i] - cy, dz = pz[i] - cz;
                const double r2 = fma(dz, dz, fma(dx, dx, dy * dy));
                // soap_weight (soap.cpp:389-420); w0 for the exact self pair,
                // the centre's own atom under the zero shift
                // (NeighborView::exact_self, neighbor.cpp:683-689).  Such an
                // image is the position plus a zero vector, so its r2 is 0
                // exactly: only rows at r2 == 0 gather the atom and shift
                double v = weight_function(a.weighting, a.w_r0, a.w_c, a.w_d, a.w_m, sqrt(r2));
                if (a.has_w0 != 0 && r2 == 0.0) {
                    const ImageDesc& image = a.images[a.bin_image[b]];
                    const bool zero = image.n[0] == 0 && image.n[1] == 0 && image.n[2] == 0;
                    if (zero && static_cast<int64_t>(a.bin_atom[b]) == c) v = a.w_w0;
                }
                row_w[row0 + r] = v * a.species_w[a.bin_type[b]];
            }
        }
    }
}

// one workgroup per structure without atoms; its row's bytes zeroed
__global__ void k_block_zero_rows(const int64_t* struct_offsets, int64_t structures, char* out, int64_t pitch,
                                  int64_t row_bytes) {
    for (int64_t s = blockIdx.x; s < structures; s += gridDim.x) {
        if (struct_offsets[s + 1] != struct_offsets[s]) continue;
        char* row = out + s * pitch;
        for (int64_t i = threadIdx.x; i < row_bytes; i += blockDim.x) row[i] = 0;
    }
}

} // namespace

void launch_block_row_weights(hipStream_t stream, const BlockArgs& a, int64_t centres, double* row_w) {
    if (centres <= 0) return;
    const unsigned grid =
        static_cast<unsigned>(std::min<int64_t>((centres + 3) / 4, 32 * static_cast<int64_t>(device_compute_units())));
    hipLaunchKernelGGL(k_block_row_weights, dim3(grid), dim3(256), 0, stream, a, centres, row_w);
    MDX_HIP(hipGetLastError());
}

void launch_block_zero_rows(hipStream_t stream, const int64_t* struct_offsets, int64_t structures, void* out,
                            int64_t pitch, int64_t row_bytes) {
    if (structures <= 0 || row_bytes <= 0) return;
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>(structures, 1 << 16));
    hipLaunchKernelGGL(k_block_zero_rows, dim3(grid), dim3(256), 0, stream, struct_offsets, structures,
                       static_cast<char*>(out), pitch, row_bytes);
    MDX_HIP(hipGetLastError());
}

} // namespace mdx
