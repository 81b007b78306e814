// Kernels 2-4 on 4x4x4 FP64 matrix-core blocks (v_mfma_f64_4x4x4f64) for the
// default SOAP options: GTO basis, no neighbour weighting, no compression, any
// average (soap.cpp:701-931, 997-1013, 1019-1142).
//
// The contraction A[(l,k)][(l,m)] = sum_j R_lk(j) Y_lm(j) (soap.cpp:893-914)
// is block-diagonal in l.  A 16x16 tile wastes most of its products on the
// zero blocks; 4x4 blocks fit the (l,k) x (l,m) blocks closely.  One
// v_mfma_f64_4x4x4f64 computes four independent 4x4 blocks, each over the
// same 4 neighbours (K = 4).  The lane layouts (measured on gfx950), with the
// block index (L/4) % 4:
//   A operand  lane L = A_b[row L % 4][k L / 16]
//   B operand  lane L = B_b[k L / 16][col L % 4]
//   result     lane L = D_b[row L / 16][col L % 4]
// so a result register is, lane for lane, a B operand: the beta fold
// c = beta A (soap.cpp:915-926) reads the contraction accumulators directly.
//
// Plan (host, plan_quad_tables): every degree l has KG = ceil(n/4) radial
// groups of 4 channels and ceil((2l+1)/4) column groups of 4 harmonics.  A
// "unit" is (l, first column group, column-group count); it occupies KG
// blocks of a register (KG = 2: blocks {0,1} or {2,3}, channel group = block
// parity; KG = 1: one block).  Each wavefront owns one register of units: its
// lanes evaluate exp(-a_lk d^2) for their block's row and the step's 4
// neighbours (one exp per lane and step), then run one MFMA per column group.
// With KG = 2 the two channel groups of a unit are summed in the fold: block
// b and b^1 exchange accumulators with one DPP row_half_mirror (lane i <->
// 7 - i inside each 8 lanes), which also reverses the column order, so the
// odd block of every unit keeps its harmonic columns reversed.  The fold of
// block b produces radial group b % 2 of the unit's c, written to LDS in the
// layout the Gram-tile power spectrum of soap_device.h reads.
#include "soap_device.h"

#include <algorithm>
#include <cmath>
#include <type_traits>
#include <utility>

namespace mdx {
namespace {

constexpr int kQuadTab = 64;  // 2^(j/64) table entries
constexpr int kYStride = kNb + 1; // harmonic staging: entry h of slot j at h * kYStride + j

__device__ inline double mfma4(double a, double b, double c) {
    return __builtin_amdgcn_mfma_f64_4x4x4f64(a, b, c, 0, 0, 0);
}

// value of lane 8*(L/8) + 7 - L%8 (DPP row_half_mirror), as a double
__device__ inline double half_mirror(double v) {
    const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(v), 0x141, 0xF, 0xF, true);
    const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(v), 0x141, 0xF, 0xF, true);
    return __hiloint2double(hi, lo);
}

// exp(-a d2) for d2 >= 0, given e1 = -a 64/ln2, by the table-driven method
// of P. T. P. Tang (ACM TOMS 15(2), 1989) with the argument reduction done
// on the product: y = d2 e1 = 64k + j + rs, |rs| <= 1/2, and
// exp(-a d2) = 2^k 2^(j/64) e^r with r = rs ln2/64; e^r - 1 by its degree-5
// Taylor polynomial in rs (truncation below 4e-17 relative).  rs comes from
// one fused multiply-add, d2 e1 - (64k + j), so its only rounding is that of
// e1: the result is within 5e-15 relative of exp(-a d2) for -a d2 >= -40 and
// as close as libm's exp of the rounded product -a * d2 further out.
//
// The table holds 2^(j/64) with (j << 14) taken off its high word, so that
// adding n << 14 (n = 64k + j, the low word of the shifted y) to that word
// multiplies by 2^k and restores the mantissa in one integer add.  The
// result must be a normal number: -a d2 >= -708, which the host checks for
// every plan that runs this kernel (kQuadMinArgument).
constexpr double kExpC1 = 0.693147180559945309417232121458176568 / 64.0; // ln2/64
constexpr double kExpC2 = kExpC1 * kExpC1 / 2.0;
constexpr double kExpC3 = kExpC2 * kExpC1 / 3.0;
constexpr double kExpC4 = kExpC3 * kExpC1 / 4.0;
constexpr double kExpC5 = kExpC4 * kExpC1 / 5.0;
__device__ __forceinline__ double exp_neg_scaled(double d2, double e1, const int2* tab) {
    constexpr double kShifter = 6755399441055744.0; // 1.5 * 2^52
    const double s = fma(d2, e1, kShifter);
    const double kf = s - kShifter;
    const double rs = fma(d2, e1, -kf);
    const int nj = __double2loint(s);
    const int2 t = *reinterpret_cast<const int2*>(reinterpret_cast<const char*>(tab) + ((nj << 3) & 0x1f8));
    double q = fma(kExpC5, rs, kExpC4);
    q = fma(q, rs, kExpC3);
    q = fma(q, rs, kExpC2);
    q = fma(q, rs, kExpC1);
    const double em1 = q * rs; // e^r - 1
    const double tk = __hiloint2double(t.y + (nj << 14), t.x); // 2^k 2^(j/64)
    return fma(tk, em1, tk);
}

// Byte offset that no output row reaches: a buffer store there is dropped by
// the buffer's range check.
constexpr int kDroppedOffset = 0x40000000;

typedef int i2 __attribute__((ext_vector_type(2)));

// Power spectrum of the coefficients in LDS (16x16 Gram tiles; units (tile
// pair, l) split over the wavefronts in contiguous ranges, as in
// power_spectrum_walk) written to one output row of F values of d.out_dtype
// bytes with raw buffer stores.  A lane's feature offsets for a tile pair come
// from the plan's fbase/fstride tables (layout of soap.cpp:997-1013); channel
// pairs i > j and pad channels get an offset past the row, which the buffer's
// range check drops, so the stores need no branches.
template <int kSteps>
__device__ __forceinline__ d4 gram_tile(const double* arow, const double* brow) {
    double a[kSteps], b[kSteps];
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
        a[s] = arow[4 * s];
        b[s] = brow[4 * s];
    }
    d4 acc = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int s = 0; s < kSteps; ++s) acc = mfma(a[s], b[s], acc);
    return acc;
}

// first column of degree l in a padded coefficient row (each degree's block
// rounded up to a multiple of 4 columns)
constexpr int padded_offset(int l) {
    int off = 0;
    for (int i = 0; i < l; ++i) off += 4 * ((2 * i + 4) / 4);
    return off;
}

// f(integral_constant<int, l>) for l = 0 .. kQuadLmax, in order
template <typename F, int... Ls>
__device__ __forceinline__ void for_each_degree(F&& f, std::integer_sequence<int, Ls...>) {
    (f(std::integral_constant<int, Ls>{}), ...);
}

template <int kBytes>
__device__ void power_spectrum_row(const double* s_c, const MfmaDims& d, const double* __restrict__ ps_pref,
                                   const int32_t* __restrict__ fbase, const int32_t* __restrict__ fstride,
                                   void* out_row, int wave, int waves) {
    const int lane = threadIdx.x % kWaveThreads;
    const int W = d.S * d.n;
    const int zero_row = d.crow - 1;
    const int RT = (W + 15) / 16;
    const int L = d.L;
    const int hp = d.cpitch;
    const int units = RT * (RT + 1) / 2 * L;
    const int u_begin = wave * units / waves;
    const int u_end = (wave + 1) * units / waves;
    constexpr int esize = kBytes;
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(out_row, 0, static_cast<int>(d.F * esize), 0x00020000);
    // the range as runs of degrees of one tile pair; within a run the
    // degrees are unrolled, so their K steps, column offsets and prefactor
    // reads are fixed at compile time and consecutive degrees' reads and
    // MFMAs overlap
    int u = u_begin;
    while (u < u_end) {
        int p = u / L;
        const int l0 = u - p * L;
        const int l1 = min(L, l0 + (u_end - u));
        int bi = 0;
        while (p >= RT - bi) {
            p -= RT - bi;
            ++bi;
        }
        const int bj = bi + p;
        const int ia = 16 * bi + lane % 16 < W ? 16 * bi + lane % 16 : zero_row;
        const int jb = 16 * bj + lane % 16 < W ? 16 * bj + lane % 16 : zero_row;
        const double* arow = s_c + ia * hp + lane / 16;
        const double* brow = s_c + jb * hp + lane / 16;
        int fb[4], fs[4];
        {
            const int j = 16 * bj + lane % 16;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = 16 * bi + lane / 16 + 4 * r;
                const int idx = i < W && j < W ? i * W + j : -1;
                const int base = idx >= 0 ? fbase[idx] : -1;
                fb[r] = base >= 0 ? base * esize : kDroppedOffset;
                fs[r] = base >= 0 ? fstride[idx] * esize : 0;
            }
        }
        auto degree = [&](auto lc) {
            constexpr int l = decltype(lc)::value;
            if (l < l0 || l >= l1) return;
            constexpr int kSteps = (2 * l + 4) / 4;
            const d4 acc4 = gram_tile<kSteps>(arow + padded_offset(l), brow + padded_offset(l));
            const double pref = ps_pref[l];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const double v = pref * acc4[r];
                const int off = fb[r] + l * fs[r];
                if (esize == 4) {
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(static_cast<float>(v)), rsrc, off, 0, 0);
                } else {
                    const i2 bits = {__double2loint(v), __double2hiint(v)};
                    __builtin_amdgcn_raw_buffer_store_b64(bits, rsrc, off, 0, 0);
                }
            }
        };
        for_each_degree(degree, std::make_integer_sequence<int, kQuadLmax + 1>{});
        u += l1 - l0;
    }
}

// KG radial groups, G MFMA instructions per step for every wavefront; the
// workgroup has blockDim.x / 64 wavefronts (one per register of the plan), at
// most kQuadMaxWaves, and keeps 5 wavefronts per SIMD (96 VGPRs): with its
// LDS footprint under 32 KB, five 4-wavefront workgroups share a CU
template <int KG, int G>
__global__ __launch_bounds__(kQuadMaxWaves * kWaveThreads) __attribute__((amdgpu_waves_per_eu(5)))
void k_soap_quad(
    const double* __restrict__ positions, const int64_t* __restrict__ pair_start, const int32_t* __restrict__ counts,
    const uint32_t* __restrict__ pair_bin, const double* __restrict__ bx, const double* __restrict__ by,
    const double* __restrict__ bz, const QuadLane* __restrict__ lanes, const double* __restrict__ ps_pref,
    const int32_t* __restrict__ fbase, const int32_t* __restrict__ fstride, MfmaDims d,
    const int64_t* __restrict__ item_begin, int64_t item_base, int64_t items, int64_t per_block, void* out,
    int64_t pitch, double* partial) {
    extern __shared__ double lds[];
    const int tid = threadIdx.x;
    const int lane = tid % kWaveThreads;
    const int kThreads = static_cast<int>(blockDim.x);
    const int T = kThreads / kWaveThreads;
    // The plan's wavefront roles carry unequal work (MFMA instructions per
    // step differ).  Wavefront w of every workgroup tends to land on the same
    // SIMD of a CU, so the roles rotate with the workgroup index: the
    // workgroups sharing a CU spread each role over its SIMDs.
    const int wave = __builtin_amdgcn_readfirstlane((tid / kWaveThreads + static_cast<int>(blockIdx.x)) % T);
    const int H = d.H, L = d.L, S = d.S, n = d.n;
    const int hp = d.hpad;          // padded c row
    const int cp = d.cpitch;        // its LDS pitch (odd)
    const int cw = d.crow * cp;     // c words (a zero row last unless S*n is a multiple of 16)
    double* s_y = lds;              // H * kYStride, harmonic-major
    double* s_d2 = s_y + H * kYStride; // kNb
    int2* s_tab = reinterpret_cast<int2*>(s_d2 + kNb); // kQuadTab biased 2^(j/64), see exp_neg_scaled
    double* s_c = s_d2 + kNb + kQuadTab; // cw
    double* s_scale = s_c + cw;     // hp: S_lm of each padded column (scaled harmonics)
    double* s_csum = s_scale + hp;  // cw (inner average only)
    int* s_loff = reinterpret_cast<int*>(s_csum + (d.mode == 1 ? cw : 0)); // L + 1

    for (int i = tid; i < kQuadTab; i += kThreads) {
        const double t = exp2(static_cast<double>(i) / kQuadTab);
        s_tab[i] = int2{__double2loint(t), __double2hiint(t) - (i << 14)};
    }
    for (int i = tid; i < cw; i += kThreads) s_c[i] = 0.0;
    for (int i = tid; i < hp; i += kThreads) {
        // column i of the padded row: degree l block at loff[l], 4 ceil((2l+1)/4) wide
        int l = 0, off = 0;
        while (l + 1 < L && off + 4 * ((2 * l + 4) / 4) <= i) {
            off += 4 * ((2 * l + 4) / 4);
            ++l;
        }
        const int c = i - off;
        s_scale[i] = c <= 2 * l ? kScaledHarmonic.s[l][c <= l ? l - c : c - l] : 0.0;
    }
    if (tid == 0) {
        int off = 0;
        for (int l = 0; l <= L; ++l) {
            s_loff[l] = off;
            off += 4 * ((2 * l + 4) / 4);
        }
    }
    __syncthreads();
    // this lane's constants (see QuadLane)
    const QuadLane& ql = lanes[wave * kWaveThreads + lane];
    const double e1 = ql.exp_scale;
    const double beta_r = ql.beta_r;
    const double beta_s = KG == 2 ? ql.beta_s : 0.0;
    // the lane's harmonic row of each instruction at its step's first slot
    const double* yrow[G];
#pragma unroll
    for (int g = 0; g < G; ++g) yrow[g] = s_y + ql.ycol[g] * kYStride + lane / 16;
    const int cdst = ql.cdst;
    const int ccount = ql.cnt;
    // MFMA instructions per step of this wavefront: its largest unit (the
    // plan pads every wavefront to G; the common path runs only these)
    int wave_instr = ccount;
#pragma unroll
    for (int off = 1; off < kWaveThreads; off *= 2) wave_instr = max(wave_instr, __shfl_xor(wave_instr, off));
    wave_instr = __builtin_amdgcn_readfirstlane(wave_instr);
    const uint32_t hmask = d.harm_mask[wave];
    const int krow = lane / 16; // neighbour of the step this lane feeds (K index)

    const int64_t item_first = item_base + static_cast<int64_t>(blockIdx.x) * per_block;
    const int64_t item_last = min(item_first + per_block, item_base + items);
    const int64_t range_end = item_first >= item_last ? 0 : item_begin ? item_begin[item_last] : item_last;
    // next centre's species row counts (lanes t, 16 + t and 32 + t for t < S),
    // position bits (lanes 0-2) and first pair row (lane 3), loaded one centre ahead
    int pre_count = 0;
    int64_t pre_bits = 0;
    auto prefetch_centre = [&](int64_t c) {
        if (c < range_end) {
            if (lane % kMaxSpecies < S && lane < 3 * kMaxSpecies) pre_count = counts[c * S + lane % kMaxSpecies];
            if (lane < 3) {
                pre_bits = __double_as_longlong(positions[c * 3 + lane]);
            } else if (lane == 3) {
                pre_bits = pair_start[c];
            }
        }
    };
    if (item_first < item_last) prefetch_centre(item_begin ? item_begin[item_first] : item_first);
    // Slot table of a centre, from pre_count.  Each species' rows fill a
    // segment of slots padded to a multiple of 4 (a step never mixes
    // species).  Lane t < S holds the first slot of species t, lane 16 + t the
    // shift from its slots to its rows, lane 32 + t the end of its rows in
    // slots; slots is the padded total and empty the bit mask of the species
    // without rows.
    int table = 0, slots = 0;
    uint32_t empty = 0;
    auto slot_table = [&]() {
        const int seg = lane / kMaxSpecies;
        int rows = seg < 3 && lane % kMaxSpecies < S ? pre_count : 0;
        const int pad = (rows + 3) & ~3;
        int rows_in = rows, pad_in = pad;
#pragma unroll
        for (int off = 1; off < kMaxSpecies; off *= 2) {
            const int r_up = __shfl_up(rows_in, off, kMaxSpecies);
            const int p_up = __shfl_up(pad_in, off, kMaxSpecies);
            if ((lane % kMaxSpecies) >= off) {
                rows_in += r_up;
                pad_in += p_up;
            }
        }
        const int start = pad_in - pad;
        table = seg == 0 ? start : seg == 1 ? start - (rows_in - rows) : start + rows;
        slots = __builtin_amdgcn_readlane(pad_in, S - 1);
        empty = static_cast<uint32_t>(__ballot(lane < S && rows == 0));
    };
    // Row of slot base + lane / 2 times 16 plus its species, or -1 for a pad
    // slot (base: the first slot of a chunk, the same in every lane).  The
    // species of slot base comes from a scan of the segment starts; only
    // segments that start inside the chunk are compared lane by lane.
    auto slot_code = [&](int base) -> int {
        int q0 = 0;
        while (q0 + 1 < S && __builtin_amdgcn_readlane(table, q0 + 1) <= base) ++q0;
        const int p = base + lane / 2;
        int q = q0;
        int shift = __builtin_amdgcn_readlane(table, kMaxSpecies + q0);
        int end = __builtin_amdgcn_readlane(table, 2 * kMaxSpecies + q0);
        for (int t = q0 + 1; t < S; ++t) {
            const int first_slot = __builtin_amdgcn_readlane(table, t);
            if (first_slot >= base + kNb) break;
            if (p >= first_slot) {
                q = t;
                shift = __builtin_amdgcn_readlane(table, kMaxSpecies + t);
                end = __builtin_amdgcn_readlane(table, 2 * kMaxSpecies + t);
            }
        }
        return p < end ? ((p - shift) << 4) | q : -1;
    };
    // lane pair jj = lane/2 holds slot jj of the current chunk: its image
    // position (stale, finite values in pad slots) and code (slot_code); of
    // the next chunk, the code and the bin of the row.  For a centre's first
    // two chunks these are loaded during the previous centre (first_ready)
    // when there was one.
    double px = 0.0, py = 0.0, pz = 0.0;
    int pcode = -1, ncode = -1;
    uint32_t nbin = 0;
    bool first_ready = false;
    for (int64_t item = item_first; item < item_last; ++item) {
        const int64_t first = item_begin ? item_begin[item] : item;
        const int64_t last = item_begin ? item_begin[item + 1] : item + 1;
        double* part_row =
            partial != nullptr ? partial + item * (d.mode == 1 ? static_cast<int64_t>(d.crow) * hp : d.F) : nullptr;
        if (d.mode == 1) {
            for (int i = tid; i < cw; i += kThreads) s_csum[i] = 0.0;
        }
        for (int64_t centre = first; centre < last; ++centre) {
            const double cx = __longlong_as_double(lane_value(pre_bits, 0));
            const double cy = __longlong_as_double(lane_value(pre_bits, 1));
            const double cz = __longlong_as_double(lane_value(pre_bits, 2));
            const int64_t centre_pairs = lane_value(pre_bits, 3);
            if (!first_ready) {
                slot_table();
                pcode = slot_code(0);
                if (pcode >= 0) {
                    const uint32_t b = pair_bin[centre_pairs + (pcode >> 4)];
                    px = bx[b];
                    py = by[b];
                    pz = bz[b];
                }
                ncode = slot_code(kNb);
                if (ncode >= 0) nbin = pair_bin[centre_pairs + (ncode >> 4)];
            }
            // the following centre's metadata, in flight during this one
            prefetch_centre(centre + 1);
            // An empty species leaves its coefficients at zero.  The previous
            // centre's power spectrum may still read s_c: the zeros are
            // written after the first barrier of this centre, which every
            // wavefront reaches only after that power spectrum.
            auto zero_empty_species = [&]() {
                for (uint32_t m = empty; m != 0; m &= m - 1) {
                    double* cdst_q = s_c + __builtin_ctz(m) * n * cp;
                    for (int i = tid; i < n * cp; i += kThreads) cdst_q[i] = 0.0;
                }
            };
            if (slots == 0) {
                __syncthreads();
                zero_empty_species();
            }
            // species of the first rows (the accumulators start there)
            const uint32_t filled = ~empty & ((2u << (S - 1)) - 1u);
            int cur = filled != 0 ? __builtin_ctz(filled) : 0;
            double acc[G];
#pragma unroll
            for (int g = 0; g < G; ++g) acc[g] = 0.0;
            // c of species q from the accumulators: c = beta A per column
            // group, the two radial groups of a unit summed through the
            // half-mirror exchange (KG = 2); instructions past a block's own
            // count summed zeros and are not stored
            auto fold = [&](int q) {
                double* cdst_q = s_c + q * n * cp + cdst;
                // the harmonics were staged in the scaled form: each output
                // column takes its S_lm (cdst is the column plus n' * cp)
                const int nrow = (KG == 2 ? 4 * ((lane / 4) % 2) : 0) + lane / 16;
                const double* scale_col = s_scale + (cdst - nrow * cp);
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    if (g >= wave_instr) break;
                    double c = mfma4(beta_r, acc[g], 0.0);
                    if (KG == 2) c = mfma4(beta_s, half_mirror(acc[g]), c);
                    if (cdst >= 0 && g < ccount) cdst_q[4 * g] = c * scale_col[4 * g];
                }
            };
            // operands of steps h and h + 1 of the chunk: exps and harmonic reads
            auto operands = [&](int h, double(&ev)[2], double(&yv)[2][G]) {
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    const int jj = 4 * (h + s) + krow;
                    ev[s] = exp_neg_scaled(s_d2[jj], e1, s_tab);
#pragma unroll
                    for (int g = 0; g < G; ++g) yv[s][g] = yrow[g][4 * (h + s)];
                }
            };
            // the steps of a chunk on the wavefront's own instruction count GW,
            // in pairs up to the end of the centre's rows (a step past it, in
            // the last pair, has slots with all-zero harmonics and adds zeros)
            auto steps_of_chunk = [&](auto gw, int nst) {
                constexpr int GW = decltype(gw)::value;
#pragma unroll
                for (int h = 0; h < kNb / 4; h += 2) {
                    if (h >= nst) break;
                    double ev[2], yv[2][GW];
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        ev[s] = exp_neg_scaled(s_d2[4 * (h + s) + krow], e1, s_tab);
#pragma unroll
                        for (int g = 0; g < GW; ++g) yv[s][g] = yrow[g][4 * (h + s)];
                    }
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
#pragma unroll
                        for (int g = 0; g < GW; ++g) acc[g] = mfma4(ev[s], yv[s][g], acc[g]);
                    }
                }
            };
            uint32_t chunk_species = 0; // species of the current chunk's steps, 4 bits each
            // A chunk whose steps within the rows all continue the current
            // species (the common case: one species' rows span several chunks,
            // and the centre's last chunk) runs without per-step checks; a
            // chunk that changes species checks each step (a fold).
            auto contract = [&](int j0) {
                const uint32_t species = chunk_species;
                const int nst = min(kNb / 4, (slots - j0) / 4);
                const uint32_t live = nst >= kNb / 4 ? 0xffffffffu : (1u << (4 * nst)) - 1u;
                if (((species ^ static_cast<uint32_t>(cur) * 0x11111111u) & live) == 0) {
                    if (G >= 4 && wave_instr >= 4) {
                        steps_of_chunk(std::integral_constant<int, (G >= 4 ? 4 : G)>{}, nst);
                    } else if (G >= 3 && wave_instr == 3) {
                        steps_of_chunk(std::integral_constant<int, (G >= 3 ? 3 : G)>{}, nst);
                    } else if (G >= 2 && wave_instr == 2) {
                        steps_of_chunk(std::integral_constant<int, (G >= 2 ? 2 : G)>{}, nst);
                    } else {
                        steps_of_chunk(std::integral_constant<int, 1>{}, nst);
                    }
                    return;
                }
#pragma unroll
                for (int h = 0; h < kNb / 4; h += 2) {
                    if (h >= nst) break;
                    double ev[2], yv[2][G];
                    operands(h, ev, yv);
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        if (h + s < nst) {
                            const int qs = static_cast<int>((species >> (4 * (h + s))) & 15u);
                            if (qs != cur) {
                                fold(cur);
                                cur = qs;
#pragma unroll
                                for (int g = 0; g < G; ++g) acc[g] = 0.0;
                            }
#pragma unroll
                            for (int g = 0; g < G; ++g) acc[g] = mfma4(ev[s], yv[s][g], acc[g]);
                        }
                    }
                }
            };
            for (int j0 = 0; j0 < slots; j0 += kNb) {
                {
                    // harmonics: two lanes per slot (cos / sin parts), this
                    // wavefront's m-columns; pad slots get all-zero harmonics.
                    // Every wavefront of the workgroup waits for the slowest
                    // at the next barrier: this phase issues ahead of other
                    // workgroups' contraction steps on the same SIMD.
                    __builtin_amdgcn_s_setprio(2);
                    const int jj = lane / 2;
                    const int comp = lane % 2;
                    const double dx = px - cx;
                    const double dy = py - cy;
                    const double dz = pz - cz;
                    const double d2 = dx * dx + dy * dy + dz * dz;
                    const double scale = pcode >= 0 ? 1.0 : 0.0;
                    // a pad slot's position is stale (an earlier row, possibly of
                    // another structure): its d2 is unbounded, so it enters the
                    // exp as 0 (its harmonics are zero)
                    if (wave == 0 && comp == 0) s_d2[jj] = pcode >= 0 ? d2 : 0.0;
                    // species of the 8 steps, 4 bits each, from the first slot
                    // of each step (lane 8 h; never a pad slot within the rows)
                    const int pq = pcode & 15;
                    chunk_species = 0;
#pragma unroll
                    for (int h = 0; h < kNb / 4; ++h) {
                        chunk_species |= static_cast<uint32_t>(__builtin_amdgcn_readlane(pq, 8 * h)) << (4 * h);
                    }
                    int lm = d.l_max, zero = 0;
                    uint32_t mk = hmask;
                    asm volatile("" : "+s"(lm), "+s"(mk), "+s"(zero));
                    int part = comp;
                    asm volatile("" : "+v"(part));
                    harmonics_scaled<0, kQuadLmax, kYStride>(dx, dy, dz, scale, lm, mk, part, &kScaledHarmonic + zero,
                                                             s_y + jj);
                }
                __syncthreads();
                __builtin_amdgcn_s_setprio(0);
                if (j0 == 0) zero_empty_species();
                {
                    // the next chunk's positions (its bin was loaded one chunk
                    // ago), then the bin of the chunk after it
                    pcode = ncode;
                    if (pcode >= 0) {
                        px = bx[nbin];
                        py = by[nbin];
                        pz = bz[nbin];
                    }
                    ncode = slot_code(j0 + 2 * kNb);
                    if (ncode >= 0) nbin = pair_bin[centre_pairs + (ncode >> 4)];
                }
                contract(j0);
                __syncthreads();
            }
            if (slots > 0) fold(cur);
            // First two chunks of the following centre: its slot table from the
            // prefetched species counts, the bins of both chunks now and the
            // image positions of the first after the power spectrum, so that
            // no load waits at the next centre's start.
            first_ready = centre + 1 < range_end;
            uint32_t next_bin = 0;
            if (first_ready) {
                const int64_t next_pairs = lane_value(pre_bits, 3);
                slot_table();
                pcode = slot_code(0);
                if (pcode >= 0) next_bin = pair_bin[next_pairs + (pcode >> 4)];
                ncode = slot_code(kNb);
                if (ncode >= 0) nbin = pair_bin[next_pairs + (ncode >> 4)];
            }
            __syncthreads();
            if (d.mode == 0) {
                char* row = static_cast<char*>(out) + centre * pitch;
                if (d.out_dtype == 4) {
                    power_spectrum_row<4>(s_c, d, ps_pref, fbase, fstride, row, wave, T);
                } else {
                    power_spectrum_row<8>(s_c, d, ps_pref, fbase, fstride, row, wave, T);
                }
            } else if (d.mode == 1) {
                for (int i = tid; i < cw; i += kThreads) s_csum[i] += s_c[i];
            } else {
                power_spectrum_tiles(s_c, s_loff, d, ps_pref, centre == first ? 3 : 2, out, pitch, centre, part_row,
                                     wave, T);
            }
            if (first_ready && pcode >= 0) {
                px = bx[next_bin];
                py = by[next_bin];
                pz = bz[next_bin];
            }
        }
        if (d.mode == 1) {
            __syncthreads(); // every thread's last s_csum update
            // partial rows at a pitch of hp (row r of s_csum starts at r * (hp + 1))
            for (int i = tid; i < d.crow * hp; i += kThreads) part_row[i] = s_csum[i + i / hp];
        }
        __syncthreads();
    }
}

template <int KG, int G>
void launch(hipStream_t stream, int waves, unsigned grid, int64_t per_block, size_t lds, const PreparedBatch& pb,
            const DeviceGraph& g, const QuadLane* lanes, const double* ps_pref, const int32_t* fbase,
            const int32_t* fstride, const MfmaDims& d, const int64_t* item_begin, int64_t base, int64_t count,
            void* out, int64_t pitch, double* partial) {
    hipLaunchKernelGGL((k_soap_quad<KG, G>), dim3(grid), dim3(waves * kWaveThreads), lds, stream,
                       pb.d_positions.as<double>(), g.pair_start.as<int64_t>(), g.counts.as<int32_t>(),
                       g.pair_bin.as<uint32_t>(), g.bin_x.as<double>(), g.bin_y.as<double>(), g.bin_z.as<double>(),
                       lanes, ps_pref, fbase, fstride, d, item_begin, base, count, per_block, out, pitch, partial);
}

template <int KG>
void launch_instr(int instr, hipStream_t stream, int waves, unsigned grid, int64_t per_block, size_t lds,
                  const PreparedBatch& pb, const DeviceGraph& g, const QuadLane* lanes, const double* ps_pref,
                  const int32_t* fbase, const int32_t* fstride, const MfmaDims& d, const int64_t* item_begin, int64_t base, int64_t count, void* out, int64_t pitch,
                  double* partial) {
    switch (instr) {
    case 1: launch<KG, 1>(stream, waves, grid, per_block, lds, pb, g, lanes, ps_pref, fbase, fstride, d, item_begin, base, count, out, pitch, partial); break;
    case 2: launch<KG, 2>(stream, waves, grid, per_block, lds, pb, g, lanes, ps_pref, fbase, fstride, d, item_begin, base, count, out, pitch, partial); break;
    case 3: launch<KG, 3>(stream, waves, grid, per_block, lds, pb, g, lanes, ps_pref, fbase, fstride, d, item_begin, base, count, out, pitch, partial); break;
    case 4: launch<KG, 4>(stream, waves, grid, per_block, lds, pb, g, lanes, ps_pref, fbase, fstride, d, item_begin, base, count, out, pitch, partial); break;
    default: throw Error(MDX_INTERNAL, "unsupported instruction count for the 4x4-block kernel");
    }
}

} // namespace

QuadPlanHost plan_quad_tables(int n, int l_max, int hpad, const std::vector<double>& beta_scaled,
                              const std::vector<double>& pref, const std::vector<double>& expo) {
    QuadPlanHost out;
    const int KG = (n + 3) / 4;
    if (KG > 2 || l_max > kQuadLmax || n < 1) return out;
    const int P = 4 / KG; // units per register
    const int L = l_max + 1;
    struct Unit {
        int l, g0, cnt;
    };
    // choose the largest column-group count per unit c (splitting degrees with
    // more groups into balanced pieces) that minimises the estimated cost of a
    // step: every wavefront evaluates one exp per lane and runs as many MFMAs
    // as the largest unit of the plan has column groups
    constexpr double kExpCost = 3.0, kMfmaCost = 1.0;
    double best_cost = 0.0;
    std::vector<std::vector<Unit>> best;
    for (int c = 1; c <= kQuadG; ++c) {
        std::vector<Unit> units;
        for (int l = 0; l < L; ++l) {
            const int groups = (2 * l + 1 + 3) / 4;
            const int pieces = (groups + c - 1) / c;
            int g0 = 0;
            for (int p = 0; p < pieces; ++p) {
                const int cnt = groups / pieces + (p < groups % pieces ? 1 : 0);
                units.push_back({l, g0, cnt});
                g0 += cnt;
            }
        }
        // pack P units per register, largest first
        std::stable_sort(units.begin(), units.end(), [](const Unit& a, const Unit& b) { return a.cnt > b.cnt; });
        std::vector<std::vector<Unit>> regs;
        for (size_t i = 0; i < units.size(); i += static_cast<size_t>(P)) {
            regs.emplace_back(units.begin() + static_cast<std::ptrdiff_t>(i),
                              units.begin() + static_cast<std::ptrdiff_t>(std::min(units.size(), i + P)));
        }
        if (regs.size() > static_cast<size_t>(kQuadMaxWaves)) continue;
        int gmax = 0;
        for (const auto& r : regs) gmax = std::max(gmax, r.front().cnt);
        const double cost = static_cast<double>(regs.size()) * (kExpCost + kMfmaCost * gmax);
        if (best.empty() || cost < best_cost) {
            best_cost = cost;
            best = regs;
        }
    }
    if (best.empty()) return out;
    const int T = static_cast<int>(best.size());
    out.waves = T;
    out.kg = KG;
    out.units.assign(static_cast<size_t>(T), 0);
    out.lanes.assign(static_cast<size_t>(T) * 64, QuadLane{});
    std::vector<int> loff(static_cast<size_t>(L) + 1, 0);
    for (int l = 0; l < L; ++l) loff[static_cast<size_t>(l) + 1] = loff[static_cast<size_t>(l)] + 4 * ((2 * l + 4) / 4);
    auto beta = [&](int l, int np, int k) -> double {
        if (np >= n || k >= n) return 0.0;
        return beta_scaled[static_cast<size_t>((l * n + np) * n + k)] * pref[static_cast<size_t>(l * n + k)];
    };
    for (int w = 0; w < T; ++w) {
        const auto& reg = best[static_cast<size_t>(w)];
        out.units[static_cast<size_t>(w)] = reg.front().cnt;
        out.instr = std::max(out.instr, reg.front().cnt);
        for (int lane = 0; lane < 64; ++lane) {
            QuadLane& q = out.lanes[static_cast<size_t>(w) * 64 + static_cast<size_t>(lane)];
            const int b = (lane / 4) % 4;
            const int slot = b / KG; // unit slot of this block
            // pad columns, idle blocks and instructions past a unit read
            // harmonic 0 (finite): the fold stores nothing for the latter two
            // and scales pad columns by an S_lm of 0
            for (int g = 0; g < kQuadG; ++g) q.ycol[g] = 0;
            q.cdst = -1;
            q.cnt = 0;
            if (slot >= static_cast<int>(reg.size())) continue; // idle block
            const Unit& u = reg[static_cast<size_t>(slot)];
            const int grp = KG == 2 ? b % 2 : 0;    // radial group of the block's A rows
            const bool reversed = KG == 2 && (b % 2) == 1;
            // A operand (exp): row lane % 4 of radial group grp
            const int k = 4 * grp + lane % 4;
            // exp_neg_scaled's e1 = -a 64/ln2, rounded once from a long double product
            q.exp_scale = k < n ? static_cast<double>(-static_cast<long double>(expo[static_cast<size_t>(u.l * n + k)])
                                                      * (64.0L / 0.693147180559945309417232121458176568L))
                                : 0.0;
            // B operand (harmonics): column lane % 4 of column group g0 + g
            const int col = lane % 4;
            const int mcol = reversed ? 3 - col : col;
            for (int g = 0; g < u.cnt; ++g) {
                const int m = 4 * (u.g0 + g) + mcol;
                q.ycol[g] = m <= 2 * u.l ? u.l * u.l + m : 0;
                // column l*l + m holds order |l - m| (cos parts first, then sin)
            }
            // fold: A operand = beta (row n' = lane % 4 of radial group grp,
            // k = lane / 16 of the block's own group, or of the partner's for
            // the exchanged accumulator); result row n' = lane / 16
            const int np_a = 4 * grp + lane % 4;
            q.beta_r = beta(u.l, np_a, 4 * grp + lane / 16);
            q.beta_s = KG == 2 ? beta(u.l, np_a, 4 * (1 - grp) + lane / 16) : 0.0;
            const int np_out = 4 * grp + lane / 16;
            if (np_out < n) {
                q.cdst = np_out * quad_coefficient_pitch(hpad) + loff[static_cast<size_t>(u.l)] + 4 * u.g0 + mcol;
                q.cnt = u.cnt;
            }
        }
    }
    return out;
}

size_t quad_lds_bytes(const MfmaDims& d) {
    const size_t cw = static_cast<size_t>(d.crow) * static_cast<size_t>(quad_coefficient_pitch(d.hpad));
    size_t words = static_cast<size_t>(d.H) * kYStride + kNb + kQuadTab + cw + d.hpad;
    if (d.mode == 1) words += cw;
    return words * sizeof(double) + static_cast<size_t>(d.L + 1) * sizeof(int);
}

void launch_quad_expand(hipStream_t stream, int waves, int kg, int instr, const PreparedBatch& pb, const DeviceGraph& g,
                        const QuadLane* lanes, const double* ps_pref, const int32_t* fbase, const int32_t* fstride,
                        const MfmaDims& d, const int64_t* item_begin, int64_t base, int64_t count, void* out,
                        int64_t pitch, double* partial) {
    if (count <= 0) return;
    const size_t lds = quad_lds_bytes(d);
    MfmaDims dm = d;
    dm.cpitch = quad_coefficient_pitch(d.hpad);
    {
        // Harmonic m-columns over the wavefronts in contiguous ranges that
        // minimise the slowest wavefront's instruction count (the barrier
        // after the harmonics waits for it).  A wavefront steps (x + iy)^m up
        // to its last column (4 instructions per step); column m costs 2
        // (its first entry), then 1 and 3 per further degree.
        const int M = d.l_max + 1;
        auto column = [&](int m) { return 2 + (m < d.l_max ? 1 + 3 * (d.l_max - m - 1) : 0); };
        auto range_cost = [&](int a, int b) { // columns a .. b-1, a < b
            int c = 4 * (b - 1);
            for (int m = a; m < b; ++m) c += column(m);
            return c;
        };
        constexpr int kInf = 1 << 30;
        // best[w][i]: least slowest cost of columns 0 .. i-1 over w wavefronts
        std::vector<std::vector<int>> best(static_cast<size_t>(waves) + 1, std::vector<int>(static_cast<size_t>(M) + 1, kInf));
        std::vector<std::vector<int>> cut(static_cast<size_t>(waves) + 1, std::vector<int>(static_cast<size_t>(M) + 1, 0));
        best[0][0] = 0;
        for (int w = 1; w <= waves; ++w) {
            for (int i = 0; i <= M; ++i) {
                for (int j = 0; j <= i; ++j) {
                    if (best[w - 1][j] == kInf) continue;
                    const int c = std::max(best[w - 1][j], j < i ? range_cost(j, i) : 0);
                    if (c < best[w][i]) {
                        best[w][i] = c;
                        cut[w][i] = j;
                    }
                }
            }
        }
        for (int w = 0; w < 16; ++w) dm.harm_mask[w] = 0;
        for (int w = waves, i = M; w >= 1; --w) {
            const int j = cut[w][i];
            for (int m = j; m < i; ++m) dm.harm_mask[w - 1] |= 1u << m;
            i = j;
        }
    }
    const int64_t resident = std::max<int64_t>(1, std::min<int64_t>(32, (160 * 1024) / std::max<size_t>(lds, 1)));
    const int64_t target = std::max<int64_t>(1, 8 * resident * device_compute_units());
    const int64_t per_block = std::max<int64_t>(1, (count + target - 1) / target);
    const unsigned grid = static_cast<unsigned>((count + per_block - 1) / per_block);
    if (waves < 1 || waves > kQuadMaxWaves) throw Error(MDX_INTERNAL, "unsupported wave count for the 4x4-block kernel");
    if (kg == 1) {
        launch_instr<1>(instr, stream, waves, grid, per_block, lds, pb, g, lanes, ps_pref, fbase, fstride, dm, item_begin,
                        base, count, out, pitch, partial);
    } else {
        launch_instr<2>(instr, stream, waves, grid, per_block, lds, pb, g, lanes, ps_pref, fbase, fstride, dm, item_begin,
                        base, count, out, pitch, partial);
    }
    MDX_HIP(hipGetLastError());
}

} // namespace mdx
