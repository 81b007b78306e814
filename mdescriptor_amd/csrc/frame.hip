// The frame: every input of kernel 1 that depends on positions, computed on
// the device at the start of each graph build.
//
// The reference builds its cell grid afresh for every structure of every
// compute call (build_grid, cpp/src/common/neighbor.cpp:135-194, called from
// build_structure_graph at :551 for each structure of compute_soap,
// cpp/src/standalone/soap.cpp:1218-1245).  Here the same grid, and what the
// device search needs beyond it, comes from the kernels below and one
// read-back of sixteen words.  A structure of at most kFuseAtoms atoms takes
// its whole frame in one wavefront (frame_small).  Larger ones are split into
// items of kItemAtoms atoms (a topology table built with the batch), one
// wavefront per item; the last item wavefront of a structure to finish
// reduces its items' partial results and does the per-structure step (no
// atomics on shared words: device atomics on one address serialise across
// the chip).
//
//   k_frame_first     one wavefront per unit: a small structure's whole
//                     frame (bounding box, grid, centres' grid coordinates,
//                     region of interest, binning path), or an item's
//                     largest and smallest coordinate per axis, the last
//                     item of a structure writing its grid (origin,
//                     dimensions, spacing from the box of its images)
//   k_frame_span      per item of a large structure: each centre's grid
//                     coordinates and their extremes, the last item
//                     classifying the structure (region of interest, binning
//                     path, LDS chunks)
//   k_lists_*         scan over the structures (one workgroup per 2,048
//                     structures and a scan of the workgroups' sums when
//                     there are more): first ROI cell of each structure, the
//                     one-cell structures' cells, the binning lists; the
//                     summary words
//   k_frame_homes     each centre's home cell and place in it; the home
//                     cells of workgroup-searched structures, listed
//                     (queued before the read-back, for the capacity the
//                     graph already holds)
//   (read-back)       the host sizes the graph and picks the launches
//   scan              first centre of each cell
//   k_frame_place     the centres grouped by home cell; each cell's structure
//
// The arithmetic is the reference's, in its order (no contraction): the
// smallest image coordinate is fl(min_j x_j + min_q s_q) because rounding is
// monotonic, so min over q of fl(min_j x_j + s_q) equals it; the padding,
// dimensions and spacing as in neighbor.cpp:159-176; coordinates as in
// CellGrid::coordinate (:122-132).  Minima and maxima are exact in any
// order.  The order of the centres inside a home cell and of the listed home
// cells follows device atomics, and nothing computed from them depends on it
// (each centre's rows go to its own slot, and a centre's rows follow the
// candidate order of its cell).
#include "mdx_internal.h"

#include <algorithm>
#include <string>

namespace mdx {
namespace {

constexpr int kFrameThreads = 256;
constexpr int kListThreads = 256;
constexpr int kListPer = 8; // consecutive structures per thread of a list workgroup

// Order key of a double: the unsigned order of keys is the order of the
// doubles (non-finite values aside; -0 sorts before +0).
__device__ inline unsigned long long order_key(double v) {
    const unsigned long long u = static_cast<unsigned long long>(__double_as_longlong(v));
    return (u >> 63) != 0 ? ~u : (u | 0x8000000000000000ull);
}

__device__ inline double from_order_key(unsigned long long k) {
    const unsigned long long u = (k >> 63) != 0 ? (k & 0x7fffffffffffffffull) : ~k;
    return __longlong_as_double(static_cast<long long>(u));
}

// Grid of one structure from its box words: origin, dimensions, spacing
// (neighbor.cpp:159-176).  bad: the reference's capacity check failed (a
// range that is not finite, or more than 1e6 cells along an axis); the grid
// is then one cell wide so that everything downstream stays in bounds until
// the host reports the error.
struct FrameGrid {
    double minimum[3];
    double spacing[3];
    int dims[3];
    bool bad;
};

__device__ inline FrameGrid frame_grid(const unsigned long long box[6], const StructGeom& g, double cutoff) {
    FrameGrid fg;
    fg.bad = false;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        const double lo = from_order_key(~box[a]);
        const double hi = from_order_key(box[3 + a]);
        double mn = lo + g.shift_lo[a];
        double mx = hi + g.shift_hi[a];
        mn -= 1e-10;
        mx += 1e-10;
        const double range = mx - mn;
        const double ncell = range / cutoff;
        if (!__builtin_isfinite(range) || range < 0.0 || !__builtin_isfinite(ncell) || ncell > 1.0e6) {
            fg.bad = true;
            fg.minimum[a] = 0.0;
            fg.dims[a] = 1;
            fg.spacing[a] = cutoff;
            continue;
        }
        fg.minimum[a] = mn;
        fg.dims[a] = max(1, static_cast<int>(ncell));
        const double width = range / fg.dims[a];
        fg.spacing[a] = cutoff < width ? width : cutoff; // std::max(cutoff, width)
    }
    return fg;
}

// Largest of v over the wavefront (butterfly).
template <typename T>
__device__ inline T wave_max(T v) {
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const T o = __shfl_xor(v, off);
        v = o > v ? o : v;
    }
    return v;
}

constexpr int kFrameWaves = kFrameThreads / kWave;

__device__ inline unsigned long long pack_cell(const uint32_t c[3]) {
    return static_cast<unsigned long long>(c[0]) | (static_cast<unsigned long long>(c[1]) << 21) |
           (static_cast<unsigned long long>(c[2]) << 42);
}

// Partial results of one item, kPartWords words: the six maxima, then (box
// words only) 1 when a coordinate was not finite.
constexpr int kPartWords = 8;

// True in the one wavefront that completes a large structure's set of items
// (the counter counts the item wavefronts done; that wavefront resets it for
// the next frame).  Its partial results are released before the count and
// everyone's acquired after it.
__device__ inline bool last_item(unsigned* done, unsigned items, int lane) {
    __threadfence();
    unsigned before = 0;
    if (lane == 0) before = atomicAdd(done, 1u);
    before = __shfl(before, 0);
    if (before + 1 != items) return false;
    __threadfence();
    if (lane == 0) *done = 0;
    return true;
}

// Largest of the items' partial words k = 0..5 (and the flag word) of large
// structure `large`, reduced over the wavefront.
template <typename T>
__device__ inline void reduce_items(const T* part, int64_t i0, int64_t i1, int lane, T v[6], T& flag) {
#pragma unroll
    for (int k = 0; k < 6; ++k) v[k] = 0;
    flag = 0;
    for (int64_t item = i0 + lane; item < i1; item += kWave) {
#pragma unroll
        for (int k = 0; k < 6; ++k) {
            const T x = part[item * kPartWords + k];
            v[k] = x > v[k] ? x : v[k];
        }
        flag = flag | part[item * kPartWords + 6];
    }
#pragma unroll
    for (int k = 0; k < 6; ++k) v[k] = wave_max(v[k]);
    flag = wave_max(flag);
}

// Class bits of a structure (classify_structure -> the list scan).
constexpr int kClassOneCell = 1;  // the ROI is one cell holding at most a wavefront of images
constexpr int kClassLds = 2;      // binned by k_bin_lds chunks (ROI of at most kLdsBinCells cells)
constexpr int kClassSmall = 4;    // binned by one wavefront of k_bin_small
constexpr int kClassLarge = 8;    // has atoms and is not small
constexpr int kClassFits = 16;    // fits one k_bin_struct workgroup
constexpr int kClassBadGrid = 32; // the grid failed the capacity check (FrameGrid::bad)
constexpr int kClassNonFinite = 64; // a position of the structure is not finite

// The region of interest (cells within one cell of a centre) of a structure
// with atoms from the span of its centres' grid coordinates (largest ~c and
// c per axis), its binning path and LDS chunks, into geom and the
// per-structure words that the list scan takes.
__device__ inline void classify_structure(StructGeom& g, const uint32_t v[6], int64_t s, int errors, int64_t* vol,
                                          int32_t* cls, int32_t* nchunks) {
    int64_t volume = 1;
    for (int a = 0; a < 3; ++a) {
        const int lo_c = static_cast<int>(~v[a]);
        const int hi_c = static_cast<int>(v[3 + a]);
        g.roi_lo[a] = max(0, lo_c - 1);
        const int hi = min(g.dims[a] - 1, hi_c + 1);
        g.roi_dim[a] = hi - g.roi_lo[a] + 1;
        volume *= g.roi_dim[a];
    }
    const int64_t images = static_cast<int64_t>(g.natoms) * g.n_images;
    const bool one_cell = volume == 1 && images <= kWaveCellImages;
    const bool lds = !one_cell && volume <= kLdsBinCells;
    const bool small = images <= kSmallImages && volume <= kSmallCells;
    const bool fits = volume <= kLdsBinCells && images <= kStructImages;
    g.one_cell = one_cell ? 1 : 0;
    g.lds_bins = lds ? 1 : 0;
    vol[s] = volume;
    cls[s] = (one_cell ? kClassOneCell : 0) | (lds ? kClassLds : 0) | (small ? kClassSmall : kClassLarge) |
             (fits ? kClassFits : 0) | errors;
    nchunks[s] = lds ? static_cast<int>((images + kBinChunk - 1) / kBinChunk) : 0;
}

// A structure without atoms: the host's defaults (one cell wide, no region
// of interest, no cells).
__device__ inline void empty_structure(StructGeom& g, int64_t s, double cutoff, int64_t* vol, int32_t* cls,
                                       int32_t* nchunks) {
    for (int a = 0; a < 3; ++a) {
        g.minimum[a] = 0.0;
        g.dims[a] = 1;
        g.spacing[a] = cutoff;
        g.roi_lo[a] = 0;
        g.roi_dim[a] = 0;
    }
    g.one_cell = 0;
    g.lds_bins = 0;
    vol[s] = 0;
    cls[s] = 0;
    nchunks[s] = 0;
}

// The whole frame of a structure of at most kFuseAtoms atoms (or none), in
// one wavefront: bounding box, grid, grid coordinates of its centres, region
// of interest and binning path, with no partial results in memory.
__device__ inline void frame_small(const double* positions, StructGeom& g, int64_t s, double cutoff, int lane,
                                   unsigned long long* atom_cell, int64_t* vol, int32_t* cls, int32_t* nchunks) {
    const int natoms = g.natoms;
    const int64_t a0 = g.atom_begin;
    if (natoms == 0) {
        if (lane == 0) empty_structure(g, s, cutoff, vol, cls, nchunks);
        return;
    }
    unsigned long long box[6] = {0ull, 0ull, 0ull, 0ull, 0ull, 0ull};
    bool finite = true;
    for (int j = lane; j < natoms; j += kWave) {
        const int64_t i = a0 + j;
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            const double p = positions[i * 3 + a];
            finite = finite && __builtin_isfinite(p);
            const unsigned long long key = order_key(p);
            box[a] = ~key > box[a] ? ~key : box[a];
            box[3 + a] = key > box[3 + a] ? key : box[3 + a];
        }
    }
    const bool all_finite = __ballot(!finite) == 0;
#pragma unroll
    for (int j = 0; j < 6; ++j) box[j] = wave_max(box[j]);
    const FrameGrid fg = frame_grid(box, g, cutoff);
    uint32_t v[6] = {0u, 0u, 0u, 0u, 0u, 0u};
    for (int j = lane; j < natoms; j += kWave) {
        const int64_t i = a0 + j;
        uint32_t c[3];
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            c[a] = static_cast<uint32_t>(grid_coordinate(positions[i * 3 + a], fg.minimum[a], fg.spacing[a],
                                                         fg.dims[a]));
            v[a] = ~c[a] > v[a] ? ~c[a] : v[a];
            v[3 + a] = c[a] > v[3 + a] ? c[a] : v[3 + a];
        }
        atom_cell[i] = pack_cell(c);
    }
#pragma unroll
    for (int j = 0; j < 6; ++j) v[j] = wave_max(v[j]);
    if (lane != 0) return;
    for (int a = 0; a < 3; ++a) {
        g.minimum[a] = fg.minimum[a];
        g.dims[a] = fg.dims[a];
        g.spacing[a] = fg.spacing[a];
    }
    classify_structure(g, v, s, (fg.bad ? kClassBadGrid : 0) | (all_finite ? 0 : kClassNonFinite), vol, cls, nchunks);
}

// First frame launch, one wavefront per unit: units [0, n_fused) are whole
// small structures (frame_small); the rest are items of the large
// structures: the largest order key of -x_a (so ~it is the smallest key of
// x_a) and of x_a, a = 0..2, and a non-finite flag, into box_part; the last
// item wavefront of a structure reduces them and writes the structure's grid
// (origin, dims, spacing) into geom.
__global__ __launch_bounds__(kFrameThreads) void k_frame_first(const double* positions, StructGeom* geom,
                                                               const int32_t* fused, int64_t n_fused,
                                                               const int32_t* large, const FrameItem* items,
                                                               int64_t n_items, const int64_t* item_start,
                                                               unsigned* done, unsigned long long* box_part,
                                                               double cutoff, unsigned long long* atom_cell,
                                                               int64_t* vol, int32_t* cls, int32_t* nchunks) {
    const int lane = threadIdx.x % kWave;
    const int64_t unit = static_cast<int64_t>(blockIdx.x) * kFrameWaves + threadIdx.x / kWave;
    if (unit < n_fused) {
        const int64_t s = fused[unit];
        frame_small(positions, geom[s], s, cutoff, lane, atom_cell, vol, cls, nchunks);
        return;
    }
    const int64_t item = unit - n_fused;
    if (item >= n_items) return;
    const FrameItem it = items[item];
    unsigned long long v[6] = {0ull, 0ull, 0ull, 0ull, 0ull, 0ull};
    bool finite = true;
#pragma unroll 4
    for (int j = lane; j < it.count; j += kWave) {
        const int64_t i = it.first + j;
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            const double p = positions[i * 3 + a];
            finite = finite && __builtin_isfinite(p);
            const unsigned long long key = order_key(p);
            v[a] = ~key > v[a] ? ~key : v[a];
            v[3 + a] = key > v[3 + a] ? key : v[3 + a];
        }
    }
    const unsigned long long flag = __ballot(!finite) != 0 ? 1ull : 0ull;
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        const unsigned long long m = wave_max(v[k]);
        if (lane == k) box_part[item * kPartWords + k] = m;
    }
    if (lane == 6) box_part[item * kPartWords + 6] = flag;
    const int64_t i0 = item_start[it.large], i1 = item_start[it.large + 1];
    if (!last_item(&done[2 * it.large], static_cast<unsigned>(i1 - i0), lane)) return;
    unsigned long long box[6], bad_position;
    reduce_items(box_part, i0, i1, lane, box, bad_position);
    if (lane != 0) return;
    const int64_t s = large[it.large];
    StructGeom& g = geom[s];
    const FrameGrid fg = frame_grid(box, g, cutoff);
    for (int a = 0; a < 3; ++a) {
        g.minimum[a] = fg.minimum[a];
        g.dims[a] = fg.dims[a];
        g.spacing[a] = fg.spacing[a];
    }
    // the error bits travel to the last span wavefront through cls
    cls[s] = (fg.bad ? kClassBadGrid : 0) | (bad_position != 0 ? kClassNonFinite : 0);
}

// Per item of a large structure: each centre's grid coordinates (kept for
// k_frame_homes), and the largest of ~c and of c per axis into span_part;
// the last item wavefront of a structure reduces them and classifies it.
__global__ __launch_bounds__(kFrameThreads) void k_frame_span(const double* positions, StructGeom* geom,
                                                              const int32_t* large, const FrameItem* items,
                                                              int64_t n_items, const int64_t* item_start,
                                                              unsigned* done, uint32_t* span_part,
                                                              unsigned long long* atom_cell, int64_t* vol,
                                                              int32_t* cls, int32_t* nchunks) {
    const int lane = threadIdx.x % kWave;
    const int64_t item = static_cast<int64_t>(blockIdx.x) * kFrameWaves + threadIdx.x / kWave;
    if (item >= n_items) return;
    const FrameItem it = items[item];
    const int64_t s = large[it.large];
    const StructGeom& g = geom[s];
    const double minimum[3] = {g.minimum[0], g.minimum[1], g.minimum[2]};
    const double spacing[3] = {g.spacing[0], g.spacing[1], g.spacing[2]};
    const int dims[3] = {g.dims[0], g.dims[1], g.dims[2]};
    uint32_t v[6] = {0u, 0u, 0u, 0u, 0u, 0u};
#pragma unroll 2
    for (int j = lane; j < it.count; j += kWave) {
        const int64_t i = it.first + j;
        uint32_t c[3];
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            c[a] = static_cast<uint32_t>(grid_coordinate(positions[i * 3 + a], minimum[a], spacing[a], dims[a]));
            v[a] = ~c[a] > v[a] ? ~c[a] : v[a];
            v[3 + a] = c[a] > v[3 + a] ? c[a] : v[3 + a];
        }
        atom_cell[i] = pack_cell(c);
    }
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        const uint32_t m = wave_max(v[k]);
        if (lane == k) span_part[item * kPartWords + k] = m;
    }
    if (lane == 6) span_part[item * kPartWords + 6] = 0u;
    const int64_t i0 = item_start[it.large], i1 = item_start[it.large + 1];
    if (!last_item(&done[2 * it.large + 1], static_cast<unsigned>(i1 - i0), lane)) return;
    uint32_t span[6], unused;
    reduce_items(span_part, i0, i1, lane, span, unused);
    if (lane != 0) return;
    const int errors = cls[s];
    classify_structure(geom[s], span, s, errors, vol, cls, nchunks);
}

// What the list scan accumulates over the structures.  Counts that cannot
// reach 2^32 share a word (high and low halves: their sums never carry
// across).
struct Tally {
    int64_t cells;        // ROI cells
    int64_t wave_small;   // one-cell structures << 32 | small structures
    int64_t chunks_large; // LDS binning chunks << 32 | large structures
    int64_t fit_direct;   // large structures that fit a binning workgroup << 32 | structures binned directly
    int64_t large_images; // images of the large structures
    int64_t big_bound;    // sum over workgroup-searched structures of min(ROI cells, atoms)
    int64_t errors;       // structures with a non-finite position << 32 | structures whose grid is too large
};
constexpr int kTallyWords = 7;
constexpr int64_t kLow = 0xffffffffll;

__device__ inline void tally_add(Tally& a, const Tally& b) {
    a.cells += b.cells;
    a.wave_small += b.wave_small;
    a.chunks_large += b.chunks_large;
    a.fit_direct += b.fit_direct;
    a.large_images += b.large_images;
    a.big_bound += b.big_bound;
    a.errors += b.errors;
}

__device__ inline int64_t& tally_word(Tally& t, int k) {
    switch (k) {
    case 0: return t.cells;
    case 1: return t.wave_small;
    case 2: return t.chunks_large;
    case 3: return t.fit_direct;
    case 4: return t.large_images;
    case 5: return t.big_bound;
    default: return t.errors;
    }
}

// Exclusive scan of a Tally over the workgroup's threads (in place); total
// receives the sums.  s_wave holds a row of kTallyWords per wavefront.
__device__ inline void block_scan(Tally& v, Tally& total, int64_t* s_wave) {
    constexpr int kWaves = kListThreads / kWave;
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    Tally incl = v;
#pragma unroll
    for (int k = 0; k < kTallyWords; ++k) {
        int64_t x = tally_word(incl, k);
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
            const int64_t u = __shfl_up(x, off);
            if (lane >= off) x += u;
        }
        tally_word(incl, k) = x;
        if (lane == kWave - 1) s_wave[wave * kTallyWords + k] = x;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kTallyWords; ++k) {
        int64_t before = 0, sum = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const int64_t x = s_wave[w * kTallyWords + k];
            before += w < wave ? x : 0;
            sum += x;
        }
        tally_word(total, k) = sum;
        tally_word(v, k) = before + tally_word(incl, k) - tally_word(v, k);
    }
    __syncthreads();
}

constexpr int64_t kListTile = static_cast<int64_t>(kListThreads) * kListPer; // structures per list workgroup

// The inputs of a thread's structures [mine, mine + kListPer), all loaded
// before anything is written (the stores to geom would otherwise order
// every later load behind them).
struct ListInputs {
    int64_t vol[kListPer];
    int32_t bits[kListPer];
    int32_t chunks[kListPer];
    int32_t natoms[kListPer];
    int32_t images[kListPer];
};

__device__ inline void load_inputs(int64_t mine, int64_t structures, const int64_t* __restrict__ vol,
                                   const int32_t* __restrict__ cls, const int32_t* __restrict__ nchunks,
                                   const StructGeom* __restrict__ geom, ListInputs& in) {
#pragma unroll
    for (int r = 0; r < kListPer; ++r) {
        const int64_t s = mine + r;
        const bool real = s < structures;
        in.vol[r] = real ? vol[s] : 0;
        in.bits[r] = real ? cls[s] : 0;
        in.chunks[r] = real ? nchunks[s] : 0;
        in.natoms[r] = real ? geom[s].natoms : 0;
        in.images[r] = real ? geom[s].n_images : 0;
    }
}

__device__ inline Tally tally_of(const ListInputs& in, int r) {
    const bool has_atoms = in.natoms[r] > 0;
    const int bits = in.bits[r];
    const bool large = (bits & kClassLarge) != 0;
    Tally t;
    t.cells = in.vol[r];
    t.wave_small = (static_cast<int64_t>((bits & kClassOneCell) != 0) << 32) | ((bits & kClassSmall) != 0 ? 1 : 0);
    t.chunks_large = (static_cast<int64_t>(in.chunks[r]) << 32) | (large ? 1 : 0);
    t.fit_direct = (static_cast<int64_t>(large && (bits & kClassFits) != 0) << 32) |
                   (has_atoms && (bits & kClassLds) == 0 ? 1 : 0);
    t.large_images = large ? static_cast<int64_t>(in.natoms[r]) * in.images[r] : 0;
    t.big_bound = has_atoms && (bits & kClassOneCell) == 0 ? min<int64_t>(in.vol[r], in.natoms[r]) : 0;
    t.errors = (static_cast<int64_t>((bits & kClassNonFinite) != 0) << 32) | ((bits & kClassBadGrid) != 0 ? 1 : 0);
    return t;
}

__device__ inline Tally thread_tally(const ListInputs& in) {
    Tally v{};
#pragma unroll
    for (int r = 0; r < kListPer; ++r) tally_add(v, tally_of(in, r));
    return v;
}

// Sums of each list workgroup's structures (more than one workgroup).
__global__ __launch_bounds__(kListThreads) void k_lists_reduce(const StructGeom* __restrict__ geom, int64_t structures,
                                                               const int64_t* __restrict__ vol,
                                                               const int32_t* __restrict__ cls,
                                                               const int32_t* __restrict__ nchunks, Tally* block_sums) {
    __shared__ int64_t s_wave[(kListThreads / kWave) * kTallyWords];
    const int64_t mine = static_cast<int64_t>(blockIdx.x) * kListTile + static_cast<int64_t>(threadIdx.x) * kListPer;
    ListInputs in;
    load_inputs(mine, structures, vol, cls, nchunks, geom, in);
    Tally v = thread_tally(in);
    Tally total{};
    block_scan(v, total, s_wave);
    if (threadIdx.x == 0) block_sums[blockIdx.x] = total;
}

// Exclusive scan of the workgroup sums (one workgroup); the total goes to
// block_sums[blocks].
__global__ __launch_bounds__(kListThreads) void k_lists_scan(Tally* block_sums, int64_t blocks) {
    __shared__ int64_t s_wave[(kListThreads / kWave) * kTallyWords];
    Tally carry{};
    for (int64_t b0 = 0; b0 < blocks; b0 += kListThreads) {
        const int64_t b = b0 + threadIdx.x;
        Tally v{};
        if (b < blocks) v = block_sums[b];
        Tally total{};
        block_scan(v, total, s_wave);
        Tally at = carry;
        tally_add(at, v);
        if (b < blocks) block_sums[b] = at;
        tally_add(carry, total);
    }
    if (threadIdx.x == 0) block_sums[blocks] = carry;
}

// Each list workgroup's structures: first ROI cell, one-cell structures'
// cells (search list head), the k_bin_small then k_bin_struct structure
// lists, the first LDS binning chunk of each structure.  With block_sums (several workgroups) each
// workgroup starts at its scanned prefix and the totals are at
// block_sums[gridDim.x]; without, the one workgroup scans everything.
// Workgroup 0 writes the summary.
__global__ __launch_bounds__(kListThreads) void k_lists_apply(StructGeom* geom, int64_t structures,
                                                              const int64_t* __restrict__ vol,
                                                              const int32_t* __restrict__ cls,
                                                              const int32_t* __restrict__ nchunks,
                                                              const Tally* __restrict__ block_sums,
                                                              int64_t* __restrict__ struct_cells,
                                                              int32_t* __restrict__ cell_lists,
                                                              int32_t* __restrict__ struct_list,
                                                              int64_t* __restrict__ struct_chunks,
                                                              unsigned long long* summary) {
    __shared__ int64_t s_wave[(kListThreads / kWave) * kTallyWords];
    const int tid = threadIdx.x;
    const int64_t mine = static_cast<int64_t>(blockIdx.x) * kListTile + static_cast<int64_t>(tid) * kListPer;
    ListInputs in;
    load_inputs(mine, structures, vol, cls, nchunks, geom, in);
    Tally v = thread_tally(in);
    Tally total{};
    block_scan(v, total, s_wave);
    Tally grand = total;
    Tally at{};
    if (block_sums != nullptr) {
        at = block_sums[blockIdx.x];
        grand = block_sums[gridDim.x];
    }
    tally_add(at, v);
    const int64_t n_small = grand.wave_small & kLow;
#pragma unroll
    for (int r = 0; r < kListPer; ++r) {
        const int64_t s = mine + r;
        if (s >= structures) continue;
        const int bits = in.bits[r];
        const int64_t cell_begin = at.cells;
        geom[s].cell_begin = cell_begin;
        struct_cells[s] = cell_begin;
        if ((bits & kClassOneCell) != 0) cell_lists[at.wave_small >> 32] = static_cast<int32_t>(cell_begin);
        struct_chunks[s] = at.chunks_large >> 32;
        if ((bits & kClassSmall) != 0) struct_list[at.wave_small & kLow] = static_cast<int32_t>(s);
        if ((bits & kClassLarge) != 0) struct_list[n_small + (at.chunks_large & kLow)] = static_cast<int32_t>(s);
        tally_add(at, tally_of(in, r));
    }
    if (blockIdx.x == 0 && tid == 0) {
        struct_cells[structures] = grand.cells;
        struct_chunks[structures] = grand.chunks_large >> 32;
        summary[kFrameStatus] = ((grand.errors >> 32) != 0 ? kFrameNonFinite : 0ull) |
                                ((grand.errors & kLow) != 0 ? kFrameGridTooLarge : 0ull);
        summary[kFrameBigCells] = 0;
        summary[kFrameCells] = static_cast<unsigned long long>(grand.cells);
        summary[kFrameWaveCells] = static_cast<unsigned long long>(grand.wave_small >> 32);
        summary[kFrameSmall] = static_cast<unsigned long long>(grand.wave_small & kLow);
        summary[kFrameChunks] = static_cast<unsigned long long>(grand.chunks_large >> 32);
        summary[kFrameLarge] = static_cast<unsigned long long>(grand.chunks_large & kLow);
        summary[kFrameLargeFit] = static_cast<unsigned long long>(grand.fit_direct >> 32);
        summary[kFrameDirect] = static_cast<unsigned long long>(grand.fit_direct & kLow);
        summary[kFrameLargeImages] = static_cast<unsigned long long>(grand.large_images);
        summary[kFrameBigBound] = static_cast<unsigned long long>(grand.big_bound);
    }
}

// Each centre's home cell and its place among the cell's centres; the first
// centre of a workgroup-searched structure's cell appends the cell to the
// search list after the one-cell structures'.  A one-cell structure's
// centres all live in its one cell, in atom order: no atomics.
// Runs before the host has read the summary: the centre counters hold
// `capacity` cells, and the kernel does nothing when the frame has more (the
// host then sizes them and runs it again).
__global__ __launch_bounds__(kFrameThreads) void k_frame_homes(const int32_t* atom_struct, int64_t atoms,
                                                               const StructGeom* geom,
                                                               const unsigned long long* atom_cell,
                                                               int32_t* centre_count, int32_t* atom_home,
                                                               int32_t* atom_rank, int32_t* cell_lists,
                                                               int64_t list_capacity, int64_t capacity,
                                                               unsigned long long* summary) {
    if (static_cast<int64_t>(summary[kFrameCells]) > capacity || summary[kFrameStatus] != 0) return;
    const int64_t wave_cells = static_cast<int64_t>(summary[kFrameWaveCells]);
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < atoms;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const StructGeom& g = geom[atom_struct[i]];
        if (g.one_cell != 0) {
            const int32_t home = static_cast<int32_t>(g.cell_begin);
            const int32_t rank = static_cast<int32_t>(i - g.atom_begin);
            if (rank == 0) centre_count[home] = g.natoms;
            atom_home[i] = home;
            atom_rank[i] = rank;
            continue;
        }
        const unsigned long long packed = atom_cell[i];
        const int cx = static_cast<int>(packed & 0x1fffffull);
        const int cy = static_cast<int>((packed >> 21) & 0x1fffffull);
        const int cz = static_cast<int>(packed >> 42);
        const int64_t local = (cx - g.roi_lo[0]) +
                              static_cast<int64_t>(g.roi_dim[0]) *
                                  ((cy - g.roi_lo[1]) + static_cast<int64_t>(g.roi_dim[1]) * (cz - g.roi_lo[2]));
        const int32_t home = static_cast<int32_t>(g.cell_begin + local);
        const int32_t rank = atomicAdd(&centre_count[home], 1);
        atom_home[i] = home;
        atom_rank[i] = rank;
        if (rank == 0) {
            const int64_t at = wave_cells + static_cast<int64_t>(atomicAdd(&summary[kFrameBigCells], 1ull));
            if (at < list_capacity) cell_lists[at] = home;
        }
    }
}

// The centres at their places (cell_centres), and the structure of every ROI
// cell: the last structure whose first cell is at or before it (structures
// without cells share their successor's first cell and are passed over).
__global__ __launch_bounds__(kFrameThreads) void k_frame_place(int64_t atoms, const int32_t* atom_home,
                                                               const int32_t* atom_rank,
                                                               const int64_t* cell_centre_start,
                                                               int32_t* cell_centres, int64_t capacity,
                                                               const int64_t* struct_cells, int64_t structures,
                                                               int32_t* cell_struct,
                                                               const unsigned long long* summary) {
    const int64_t cells = static_cast<int64_t>(summary[kFrameCells]);
    if (cells > capacity || summary[kFrameStatus] != 0) return;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    const int64_t first = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    for (int64_t i = first; i < atoms; i += stride) {
        cell_centres[cell_centre_start[atom_home[i]] + atom_rank[i]] = static_cast<int32_t>(i);
    }
    for (int64_t c = first; c < cells; c += stride) {
        int64_t lo = 0, hi = structures;
        while (hi - lo > 1) {
            const int64_t mid = (lo + hi) / 2;
            if (struct_cells[mid] <= c) lo = mid; else hi = mid;
        }
        cell_struct[c] = static_cast<int32_t>(lo);
    }
}

unsigned frame_grid_size(int64_t work) {
    return static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>((work + kFrameThreads - 1) / kFrameThreads,
                                                                        int64_t(1) << 16)));
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

} // namespace

void size_frame(PreparedBatch& pb) {
    const size_t S = static_cast<size_t>(pb.structures);
    const size_t atoms = static_cast<size_t>(pb.atoms);
    const size_t items = std::max<size_t>(1, pb.frame_items.size());
    const size_t large = pb.frame_large.size();
    const size_t blocks = (S + kListTile - 1) / kListTile;
    size_t at = align256(items * kPartWords * sizeof(unsigned long long));
    pb.frame_span = at;
    at += align256(items * kPartWords * sizeof(uint32_t));
    pb.frame_vol = at;
    at += align256(S * sizeof(int64_t));
    pb.frame_cls = at;
    at += align256(S * sizeof(int32_t));
    pb.frame_nch = at;
    at += align256(S * sizeof(int32_t));
    pb.frame_blocks = at;
    at += align256((blocks + 1) * sizeof(Tally));
    pb.frame_done = at;
    at += align256(std::max<size_t>(1, 2 * large) * sizeof(unsigned));
    pb.frame_summary = at;
    at += align256(kFrameWords * sizeof(unsigned long long));
    pb.frame_bytes = at;
    pb.d_frame.reserve(pb.frame_bytes);
    pb.d_frame_items.reserve(items * sizeof(FrameItem));
    pb.d_frame_item_start.reserve(pb.frame_item_start.size() * sizeof(int64_t));
    pb.d_frame_lists.reserve(std::max<size_t>(1, S) * sizeof(int32_t));
    pb.d_struct_cells.reserve((S + 1) * sizeof(int64_t));
    pb.d_struct_chunks.reserve((S + 1) * sizeof(int64_t));
    pb.d_cell_lists.reserve(std::max<size_t>(1, S + atoms) * sizeof(int32_t));
    pb.d_struct_list.reserve(std::max<size_t>(1, S) * sizeof(int32_t));
    pb.d_cell_centres.reserve(std::max<size_t>(1, atoms) * sizeof(int32_t));
    pb.d_atom_cell.reserve(std::max<size_t>(1, atoms) * sizeof(unsigned long long));
    pb.d_atom_home.reserve(std::max<size_t>(1, atoms) * sizeof(int32_t));
    pb.d_atom_rank.reserve(std::max<size_t>(1, atoms) * sizeof(int32_t));
    pb.frame_host.get(kFrameWords);
    pb.frame_read.prepare();
    pb.frame_done_clear = false;
}

void frame_items(PreparedBatch& pb) {
    pb.frame_items.clear();
    pb.frame_fused.clear();
    pb.frame_large.clear();
    pb.frame_item_start.assign(1, 0);
    for (int64_t s = 0; s < pb.structures; ++s) {
        const int64_t begin = pb.offsets[static_cast<size_t>(s)], end = pb.offsets[static_cast<size_t>(s) + 1];
        if (end - begin <= kFuseAtoms) {
            pb.frame_fused.push_back(static_cast<int32_t>(s));
            continue;
        }
        const int32_t k = static_cast<int32_t>(pb.frame_large.size());
        pb.frame_large.push_back(static_cast<int32_t>(s));
        for (int64_t a = begin; a < end; a += kItemAtoms) {
            pb.frame_items.push_back(
                FrameItem{a, k, static_cast<int32_t>(std::min<int64_t>(kItemAtoms, end - a))});
        }
        pb.frame_item_start.push_back(static_cast<int64_t>(pb.frame_items.size()));
    }
}

namespace {

// The centres grouped by home cell and the structure of every ROI cell, into
// the graph's arrays of `capacity` cells (k_frame_homes and k_frame_place do
// nothing when the frame has more cells or an error).  centre_count: zeroed
// counters of capacity + 1 cells.
void launch_homes(hipStream_t stream, const PreparedBatch& pb, DeviceGraph& gr, int32_t* centre_count,
                  int64_t capacity, unsigned long long* summary) {
    const int64_t atoms = pb.atoms;
    hipLaunchKernelGGL(k_frame_homes, dim3(frame_grid_size(atoms)), dim3(kFrameThreads), 0, stream,
                       pb.d_atom_struct.as<int32_t>(), atoms, pb.d_geom.as<StructGeom>(),
                       pb.d_atom_cell.as<unsigned long long>(), centre_count, pb.d_atom_home.as<int32_t>(),
                       pb.d_atom_rank.as<int32_t>(), pb.d_cell_lists.as<int32_t>(), pb.structures + atoms, capacity,
                       summary);
    scan_counts(stream, centre_count, gr.cell_centre_start.as<int64_t>(), capacity, gr.scan_tmp);
    hipLaunchKernelGGL(k_frame_place, dim3(frame_grid_size(std::max(atoms, capacity))), dim3(kFrameThreads), 0,
                       stream, atoms, pb.d_atom_home.as<int32_t>(), pb.d_atom_rank.as<int32_t>(),
                       gr.cell_centre_start.as<int64_t>(), pb.d_cell_centres.as<int32_t>(), capacity,
                       pb.d_struct_cells.as<int64_t>(), pb.structures, gr.cell_struct.as<int32_t>(), summary);
}

} // namespace

size_t graph_counter_bytes(int64_t capacity) {
    return align256(kStatWords * sizeof(unsigned long long) + 3 * static_cast<size_t>(capacity + 1) * sizeof(int32_t));
}

void reserve_cells(DeviceGraph& gr, int64_t capacity) {
    gr.counters.reserve(graph_counter_bytes(capacity));
    gr.cell_centre_start.reserve(static_cast<size_t>(capacity + 1) * sizeof(int64_t));
    gr.cell_struct.reserve(std::max<size_t>(1, static_cast<size_t>(capacity)) * sizeof(int32_t));
}

void prepare_frame(hipStream_t stream, PreparedBatch& pb, DeviceGraph& gr) {
    const int64_t S = pb.structures, atoms = pb.atoms;
    pb.cells_total = pb.wave_cells = pb.big_bound = pb.chunks = pb.small_structs = pb.large_structs = 0;
    pb.direct_bins = pb.struct_bins = false;
    if (S == 0 || atoms == 0) return;
    const int64_t n_items = static_cast<int64_t>(pb.frame_items.size());
    char* base = static_cast<char*>(pb.d_frame.ptr);
    auto* box = reinterpret_cast<unsigned long long*>(base);
    auto* span = reinterpret_cast<uint32_t*>(base + pb.frame_span);
    auto* vol = reinterpret_cast<int64_t*>(base + pb.frame_vol);
    auto* cls = reinterpret_cast<int32_t*>(base + pb.frame_cls);
    auto* nch = reinterpret_cast<int32_t*>(base + pb.frame_nch);
    auto* block_sums = reinterpret_cast<Tally*>(base + pb.frame_blocks);
    auto* done = reinterpret_cast<unsigned*>(base + pb.frame_done);
    auto* summary = reinterpret_cast<unsigned long long*>(base + pb.frame_summary);
    StructGeom* geom = pb.d_geom.as<StructGeom>();
    const double* pos = pb.d_positions.as<double>();
    const FrameItem* items = pb.d_frame_items.as<FrameItem>();
    const int64_t* item_start = pb.d_frame_item_start.as<int64_t>();
    const int64_t n_fused = static_cast<int64_t>(pb.frame_fused.size());
    const int32_t* fused = pb.d_frame_lists.as<int32_t>();
    const int32_t* large = fused + n_fused;
    const int64_t blocks = (S + kListTile - 1) / kListTile;
    if (!pb.frame_done_clear) {
        // the item wavefronts' counters: cleared once, then reset by the
        // wavefront that completes each structure
        MDX_HIP(hipMemsetAsync(done, 0, pb.frame_summary - pb.frame_done, stream));
        pb.frame_done_clear = true;
    }
    const int64_t units = n_fused + n_items;
    hipLaunchKernelGGL(k_frame_first, dim3(static_cast<unsigned>((units + kFrameWaves - 1) / kFrameWaves)),
                       dim3(kFrameThreads), 0, stream, pos, geom, fused, n_fused, large, items, n_items, item_start,
                       done, box, pb.cutoff, pb.d_atom_cell.as<unsigned long long>(), vol, cls, nch);
    if (n_items > 0) {
        hipLaunchKernelGGL(k_frame_span, dim3(static_cast<unsigned>((n_items + kFrameWaves - 1) / kFrameWaves)),
                           dim3(kFrameThreads), 0, stream, pos, geom, large, items, n_items, item_start, done, span,
                           pb.d_atom_cell.as<unsigned long long>(), vol, cls, nch);
    }
    if (blocks > 1) {
        hipLaunchKernelGGL(k_lists_reduce, dim3(static_cast<unsigned>(blocks)), dim3(kListThreads), 0, stream, geom, S,
                           vol, cls, nch, block_sums);
        hipLaunchKernelGGL(k_lists_scan, dim3(1), dim3(kListThreads), 0, stream, block_sums, blocks);
    }
    hipLaunchKernelGGL(k_lists_apply, dim3(static_cast<unsigned>(blocks)), dim3(kListThreads), 0, stream, geom, S, vol,
                       cls, nch, blocks > 1 ? block_sums : static_cast<const Tally*>(nullptr),
                       pb.d_struct_cells.as<int64_t>(), pb.d_cell_lists.as<int32_t>(), pb.d_struct_list.as<int32_t>(),
                       pb.d_struct_chunks.as<int64_t>(), summary);
    // with cells for the last frame's grid already in the graph, the centres
    // are grouped before the summary comes back (kernels that find more
    // cells in this frame do nothing, and the host repeats them below)
    int64_t capacity = gr.cell_capacity;
    if (capacity > 0) {
        reserve_cells(gr, capacity);
        MDX_HIP(hipMemsetAsync(gr.counters.ptr, 0, graph_counter_bytes(capacity), stream));
        launch_homes(stream, pb, gr, graph_centre_counts(gr, capacity), capacity, summary);
    }
    MDX_HIP(hipGetLastError());
    unsigned long long* host = pb.frame_host.get(kFrameWords);
    MDX_HIP(hipMemcpyAsync(host, summary, kFrameWords * sizeof(unsigned long long), hipMemcpyDeviceToHost, stream));
    // the graph's sizes and launches wait on these words
    pb.frame_read.wait(stream);
    const unsigned long long status = host[kFrameStatus];
    // the checks of the host's former grid preparation, in the reference's
    // order: positions (batch.hpp:71-77), then the grid (neighbor.cpp:159-176)
    if ((status & kFrameNonFinite) != 0) throw Error(MDX_INVALID_ARGUMENT, "positions must be finite");
    if ((status & kFrameGridTooLarge) != 0) {
        throw Error(MDX_INVALID_ARGUMENT, "neighbor cell-grid dimension exceeds the device graph capacity");
    }
    const int64_t cells = static_cast<int64_t>(host[kFrameCells]);
    if (cells > (int64_t(1) << 30)) throw Error(MDX_INVALID_ARGUMENT, "neighbor cell-grid exceeds the device graph capacity");
    pb.cells_total = cells;
    pb.wave_cells = static_cast<int64_t>(host[kFrameWaveCells]);
    pb.chunks = static_cast<int64_t>(host[kFrameChunks]);
    pb.small_structs = static_cast<int64_t>(host[kFrameSmall]);
    pb.large_structs = static_cast<int64_t>(host[kFrameLarge]);
    pb.big_bound = static_cast<int64_t>(host[kFrameBigBound]);
    pb.direct_bins = host[kFrameDirect] > 0;
    const int64_t fit = static_cast<int64_t>(host[kFrameLargeFit]);
    const int64_t large_images = static_cast<int64_t>(host[kFrameLargeImages]);
    pb.struct_bins = fit == pb.large_structs && pb.small_structs + pb.large_structs > 0 &&
                     large_images >= static_cast<int64_t>(kStructMinImages) * pb.large_structs;
    if (pb.chunks > pb.chunk_bound || pb.wave_cells > S || pb.small_structs + pb.large_structs > S) {
        throw Error(MDX_INTERNAL, "frame summary out of range");
    }
    if (cells > capacity) {
        // the graph's cell arrays were too small for this frame (or absent):
        // room for a quarter more, then the centres again
        capacity = cells + cells / 4 + 64;
        gr.cell_capacity = capacity;
        reserve_cells(gr, capacity);
        MDX_HIP(hipMemsetAsync(gr.counters.ptr, 0, graph_counter_bytes(capacity), stream));
        launch_homes(stream, pb, gr, graph_centre_counts(gr, capacity), capacity, summary);
        MDX_HIP(hipGetLastError());
    }
}

} // namespace mdx
