// The frame: every input of kernel 1 that depends on positions, computed on
// the device at the start of each graph build.
//
// The reference builds its cell grid afresh for every structure of every
// compute call (build_grid, cpp/src/common/neighbor.cpp:135-194, called from
// build_structure_graph at :551 for each structure of compute_soap,
// cpp/src/standalone/soap.cpp:1218-1245).  Here the same grid, and what the
// device search needs beyond it, comes from five kernels and one read-back of
// sixteen words:
//
//   k_frame_bounds    bounding box of each structure's atoms (order keys,
//                     one device atomic per structure run of a wavefront)
//   k_frame_span      each centre's grid coordinates; per structure their
//                     smallest and largest (the region of interest)
//   k_frame_classify  per structure: grid origin, dimensions and spacing,
//                     region of interest, binning path, LDS chunks
//   k_frame_lists     one workgroup scans the structures: first ROI cell of
//                     each, the one-cell structures' cells, the binning
//                     lists; the summary words
//   (read-back)       the host sizes the graph and picks the launches
//   k_frame_homes     each centre's home cell and place in it; the home
//                     cells of workgroup-searched structures, listed
//   scan              first centre of each cell
//   k_frame_place     the centres grouped by home cell; each cell's structure
//
// The arithmetic is the reference's, in its order (no contraction): the
// smallest image coordinate is fl(min_j x_j + min_q s_q) because rounding is
// monotonic, so min over q of fl(min_j x_j + s_q) equals it; the padding,
// dimensions and spacing as in neighbor.cpp:159-176; coordinates as in
// CellGrid::coordinate (:122-132).  Order keys make every min and max exact,
// whatever order the atomics land in; the order of the centres inside a home
// cell and of the listed home cells follows the atomics, and nothing computed
// from them depends on it (each centre's rows go to its own slot, rows
// follow the candidate order of its cell).
#include "mdx_internal.h"

#include <algorithm>
#include <string>

namespace mdx {
namespace {

constexpr int kFrameThreads = 256;
constexpr int kListThreads = 1024;
constexpr int kListPer = 4; // consecutive structures per thread in one pass of k_frame_lists

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

// Largest v over the lanes at or above this one that carry the same segment
// id; segments are runs of consecutive lanes (atoms are grouped by
// structure), so the first lane of a run receives the run's largest value.
template <typename T>
__device__ inline T segment_max(T v, int sid, int lane) {
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const T o = __shfl_down(v, off);
        const int os = __shfl_down(sid, off);
        if (lane + off < kWave && os == sid && o > v) v = o;
    }
    return v;
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

__device__ inline FrameGrid frame_grid(const unsigned long long* box, const StructGeom& g, double cutoff) {
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

// Bounding box of each structure's atoms as order keys: box[s*6 + a] is the
// largest key of -x_a (so ~it is the smallest key of x_a), box[s*6 + 3 + a]
// the largest key of x_a.  Zero (cleared) means no atom.
__global__ __launch_bounds__(kFrameThreads) void k_frame_bounds(const double* positions, const int32_t* atom_struct,
                                                                int64_t atoms, unsigned long long* box,
                                                                unsigned long long* summary) {
    const int lane = threadIdx.x % kWave;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t base = static_cast<int64_t>(blockIdx.x) * blockDim.x; base < atoms; base += stride) {
        const int64_t i = base + threadIdx.x;
        const bool real = i < atoms;
        const int sid = real ? atom_struct[i] : -1;
        double p[3] = {0.0, 0.0, 0.0};
        if (real) {
            p[0] = positions[i * 3 + 0];
            p[1] = positions[i * 3 + 1];
            p[2] = positions[i * 3 + 2];
            if (!__builtin_isfinite(p[0]) || !__builtin_isfinite(p[1]) || !__builtin_isfinite(p[2])) {
                atomicOr(&summary[kFrameStatus], kFrameNonFinite);
            }
        }
        const int prev = __shfl_up(sid, 1);
        const bool head = real && (lane == 0 || prev != sid);
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            const unsigned long long key = real ? order_key(p[a]) : 0ull;
            const unsigned long long lo = segment_max(real ? ~key : 0ull, sid, lane);
            const unsigned long long hi = segment_max(key, sid, lane);
            if (head) {
                atomicMax(&box[static_cast<int64_t>(sid) * 6 + a], lo);
                atomicMax(&box[static_cast<int64_t>(sid) * 6 + 3 + a], hi);
            }
        }
    }
}

// Each centre's grid coordinates (kept for k_frame_homes) and, per structure,
// their smallest (as ~c) and largest, for the region of interest.
__global__ __launch_bounds__(kFrameThreads) void k_frame_span(const double* positions, const int32_t* atom_struct,
                                                              int64_t atoms, const StructGeom* geom,
                                                              const unsigned long long* box, double cutoff,
                                                              uint32_t* span, unsigned long long* atom_cell) {
    const int lane = threadIdx.x % kWave;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t base = static_cast<int64_t>(blockIdx.x) * blockDim.x; base < atoms; base += stride) {
        const int64_t i = base + threadIdx.x;
        const bool real = i < atoms;
        const int sid = real ? atom_struct[i] : -1;
        uint32_t c[3] = {0u, 0u, 0u};
        if (real) {
            const FrameGrid fg = frame_grid(box + static_cast<int64_t>(sid) * 6, geom[sid], cutoff);
#pragma unroll
            for (int a = 0; a < 3; ++a) {
                c[a] = static_cast<uint32_t>(grid_coordinate(positions[i * 3 + a], fg.minimum[a], fg.spacing[a],
                                                              fg.dims[a]));
            }
            atom_cell[i] = static_cast<unsigned long long>(c[0]) | (static_cast<unsigned long long>(c[1]) << 21) |
                           (static_cast<unsigned long long>(c[2]) << 42);
        }
        const int prev = __shfl_up(sid, 1);
        const bool head = real && (lane == 0 || prev != sid);
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            const uint32_t lo = segment_max(real ? ~c[a] : 0u, sid, lane);
            const uint32_t hi = segment_max(c[a], sid, lane);
            if (head) {
                atomicMax(&span[static_cast<int64_t>(sid) * 6 + a], lo);
                atomicMax(&span[static_cast<int64_t>(sid) * 6 + 3 + a], hi);
            }
        }
    }
}

// Class bits of a structure (k_frame_classify -> k_frame_lists).
constexpr int kClassOneCell = 1;  // the ROI is one cell holding at most a wavefront of images
constexpr int kClassLds = 2;      // binned by k_bin_lds chunks (ROI of at most kLdsBinCells cells)
constexpr int kClassSmall = 4;    // binned by one wavefront of k_bin_small
constexpr int kClassLarge = 8;    // has atoms and is not small
constexpr int kClassFits = 16;    // fits one k_bin_struct workgroup

// Per structure: the grid, the region of interest (cells within one cell of a
// centre), the binning path; the ROI cell count, class bits and LDS chunks go
// to the per-structure words that k_frame_lists scans.
__global__ __launch_bounds__(kFrameThreads) void k_frame_classify(StructGeom* geom, int64_t structures,
                                                                  const unsigned long long* box, const uint32_t* span,
                                                                  double cutoff, int64_t* vol, int32_t* cls,
                                                                  int32_t* nchunks, unsigned long long* summary) {
    for (int64_t s = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; s < structures;
         s += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        StructGeom& g = geom[s];
        int64_t volume = 0;
        int bits = 0, chunks = 0;
        if (g.natoms == 0) {
            for (int a = 0; a < 3; ++a) {
                g.minimum[a] = 0.0;
                g.dims[a] = 1;
                g.spacing[a] = cutoff;
                g.roi_lo[a] = 0;
                g.roi_dim[a] = 0;
            }
            g.one_cell = 0;
            g.lds_bins = 0;
        } else {
            const FrameGrid fg = frame_grid(box + s * 6, g, cutoff);
            if (fg.bad) atomicOr(&summary[kFrameStatus], kFrameGridTooLarge);
            volume = 1;
            for (int a = 0; a < 3; ++a) {
                g.minimum[a] = fg.minimum[a];
                g.dims[a] = fg.dims[a];
                g.spacing[a] = fg.spacing[a];
                const int lo_c = static_cast<int>(~span[s * 6 + a]);
                const int hi_c = static_cast<int>(span[s * 6 + 3 + a]);
                g.roi_lo[a] = max(0, lo_c - 1);
                const int hi = min(fg.dims[a] - 1, hi_c + 1);
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
            chunks = lds ? static_cast<int>((images + kBinChunk - 1) / kBinChunk) : 0;
            bits = (one_cell ? kClassOneCell : 0) | (lds ? kClassLds : 0) | (small ? kClassSmall : kClassLarge) |
                   (fits ? kClassFits : 0);
        }
        vol[s] = volume;
        cls[s] = bits;
        nchunks[s] = chunks;
    }
}

// The tallies k_frame_lists scans over the structures; the first five give
// each structure its places, the rest are totals.
enum Tally {
    kTCells = 0, kTWave, kTChunks, kTSmall, kTLarge, kTFit, kTLargeImages, kTDirect, kTBigBound, kTallies
};

__device__ inline void tally_of(int64_t volume, int bits, int chunks, const StructGeom& g, int64_t t[kTallies]) {
    const bool has_atoms = g.natoms > 0;
    const bool large = (bits & kClassLarge) != 0;
    t[kTCells] = volume;
    t[kTWave] = (bits & kClassOneCell) != 0 ? 1 : 0;
    t[kTChunks] = chunks;
    t[kTSmall] = (bits & kClassSmall) != 0 ? 1 : 0;
    t[kTLarge] = large ? 1 : 0;
    t[kTFit] = large && (bits & kClassFits) != 0 ? 1 : 0;
    t[kTLargeImages] = large ? static_cast<int64_t>(g.natoms) * g.n_images : 0;
    t[kTDirect] = has_atoms && (bits & kClassLds) == 0 ? 1 : 0;
    t[kTBigBound] = has_atoms && (bits & kClassOneCell) == 0 ? min<int64_t>(volume, g.natoms) : 0;
}

// Exclusive scan of kTallies values over the workgroup's threads; total
// receives the sums.  s_wave holds kListThreads / kWave rows of kTallies.
__device__ inline void block_scan_tallies(int64_t v[kTallies], int64_t total[kTallies], int64_t* s_wave) {
    constexpr int kWaves = kListThreads / kWave;
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    int64_t incl[kTallies];
#pragma unroll
    for (int k = 0; k < kTallies; ++k) {
        int64_t x = v[k];
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
            const int64_t u = __shfl_up(x, off);
            if (lane >= off) x += u;
        }
        incl[k] = x;
        if (lane == kWave - 1) s_wave[wave * kTallies + k] = x;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kTallies; ++k) {
        int64_t before = 0, sum = 0;
        for (int w = 0; w < kWaves; ++w) {
            const int64_t x = s_wave[w * kTallies + k];
            if (w < wave) before += x;
            sum += x;
        }
        total[k] = sum;
        v[k] = before + incl[k] - v[k];
    }
    __syncthreads();
}

// One workgroup over all structures: each structure's first ROI cell, the
// one-cell structures' cells (search list head), the k_bin_small then
// k_bin_struct structure lists, the LDS binning chunks, and the summary.
__global__ __launch_bounds__(kListThreads) void k_frame_lists(StructGeom* geom, int64_t structures, const int64_t* vol,
                                                              const int32_t* cls, const int32_t* nchunks,
                                                              int64_t* struct_cells, int32_t* cell_lists,
                                                              int32_t* struct_list, BinChunk* chunks,
                                                              unsigned long long* summary) {
    __shared__ int64_t s_wave[(kListThreads / kWave) * kTallies];
    __shared__ int64_t s_small;
    const int tid = threadIdx.x;
    // small structures come first in the structure list
    {
        int64_t mine = 0;
        for (int64_t s = tid; s < structures; s += kListThreads) mine += (cls[s] & kClassSmall) != 0 ? 1 : 0;
        int64_t v[kTallies] = {}, total[kTallies];
        v[kTSmall] = mine;
        block_scan_tallies(v, total, s_wave);
        if (tid == 0) s_small = total[kTSmall];
        __syncthreads();
    }
    const int64_t n_small = s_small;
    int64_t carry[kTallies] = {};
    constexpr int64_t kTile = static_cast<int64_t>(kListThreads) * kListPer;
    for (int64_t first = 0; first < structures; first += kTile) {
        const int64_t mine = first + static_cast<int64_t>(tid) * kListPer;
        int64_t v[kTallies] = {};
        for (int r = 0; r < kListPer; ++r) {
            const int64_t s = mine + r;
            if (s >= structures) break;
            int64_t t[kTallies];
            tally_of(vol[s], cls[s], nchunks[s], geom[s], t);
            for (int k = 0; k < kTallies; ++k) v[k] += t[k];
        }
        int64_t total[kTallies];
        block_scan_tallies(v, total, s_wave);
        int64_t at[kTallies];
        for (int k = 0; k < kTallies; ++k) at[k] = carry[k] + v[k];
        for (int r = 0; r < kListPer; ++r) {
            const int64_t s = mine + r;
            if (s >= structures) break;
            StructGeom& g = geom[s];
            const int bits = cls[s];
            const int64_t cell_begin = at[kTCells];
            g.cell_begin = cell_begin;
            struct_cells[s] = cell_begin;
            if ((bits & kClassOneCell) != 0) cell_lists[at[kTWave]] = static_cast<int32_t>(cell_begin);
            const int n_ch = nchunks[s];
            const int64_t images = static_cast<int64_t>(g.natoms) * g.n_images;
            for (int k = 0; k < n_ch; ++k) {
                const int64_t from = static_cast<int64_t>(k) * kBinChunk;
                chunks[at[kTChunks] + k] = BinChunk{from, static_cast<int32_t>(s),
                                                    static_cast<int32_t>(min<int64_t>(kBinChunk, images - from))};
            }
            if ((bits & kClassSmall) != 0) struct_list[at[kTSmall]] = static_cast<int32_t>(s);
            if ((bits & kClassLarge) != 0) struct_list[n_small + at[kTLarge]] = static_cast<int32_t>(s);
            int64_t t[kTallies];
            tally_of(vol[s], bits, n_ch, g, t);
            for (int k = 0; k < kTallies; ++k) at[k] += t[k];
        }
        for (int k = 0; k < kTallies; ++k) carry[k] += total[k];
    }
    if (tid == 0) {
        struct_cells[structures] = carry[kTCells];
        summary[kFrameCells] = static_cast<unsigned long long>(carry[kTCells]);
        summary[kFrameWaveCells] = static_cast<unsigned long long>(carry[kTWave]);
        summary[kFrameChunks] = static_cast<unsigned long long>(carry[kTChunks]);
        summary[kFrameSmall] = static_cast<unsigned long long>(carry[kTSmall]);
        summary[kFrameLarge] = static_cast<unsigned long long>(carry[kTLarge]);
        summary[kFrameLargeFit] = static_cast<unsigned long long>(carry[kTFit]);
        summary[kFrameLargeImages] = static_cast<unsigned long long>(carry[kTLargeImages]);
        summary[kFrameDirect] = static_cast<unsigned long long>(carry[kTDirect]);
        summary[kFrameBigBound] = static_cast<unsigned long long>(carry[kTBigBound]);
    }
}

// Each centre's home cell and its place among the cell's centres (taken from
// the cell's counter); the first centre of a workgroup-searched structure's
// cell appends the cell to the search list after the one-cell structures'.
__global__ __launch_bounds__(kFrameThreads) void k_frame_homes(const int32_t* atom_struct, int64_t atoms,
                                                               const StructGeom* geom,
                                                               const unsigned long long* atom_cell,
                                                               int32_t* centre_count, int32_t* atom_home,
                                                               int32_t* atom_rank, int32_t* cell_lists,
                                                               int64_t wave_cells, int64_t list_capacity,
                                                               unsigned long long* summary) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < atoms;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const StructGeom& g = geom[atom_struct[i]];
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
        if (rank == 0 && g.one_cell == 0) {
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
                                                               int32_t* cell_centres, int64_t cells,
                                                               const int64_t* struct_cells, int64_t structures,
                                                               int32_t* cell_struct) {
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
    size_t at = align256(S * 6 * sizeof(unsigned long long));
    pb.frame_span = at;
    at += align256(S * 6 * sizeof(uint32_t));
    pb.frame_vol = at;
    at += align256(S * sizeof(int64_t));
    pb.frame_cls = at;
    at += align256(S * sizeof(int32_t));
    pb.frame_nch = at;
    at += align256(S * sizeof(int32_t));
    pb.frame_summary = at;
    at += align256(kFrameWords * sizeof(unsigned long long));
    pb.frame_bytes = at;
    pb.d_frame.reserve(pb.frame_bytes);
    pb.d_struct_cells.reserve((S + 1) * sizeof(int64_t));
    pb.d_cell_lists.reserve(std::max<size_t>(1, S + atoms) * sizeof(int32_t));
    pb.d_struct_list.reserve(std::max<size_t>(1, S) * sizeof(int32_t));
    pb.d_bin_chunks.reserve(std::max<size_t>(1, static_cast<size_t>(pb.chunk_bound)) * sizeof(BinChunk));
    pb.d_cell_centres.reserve(std::max<size_t>(1, atoms) * sizeof(int32_t));
    pb.d_atom_cell.reserve(std::max<size_t>(1, atoms) * sizeof(unsigned long long));
    pb.d_atom_home.reserve(std::max<size_t>(1, atoms) * sizeof(int32_t));
    pb.d_atom_rank.reserve(std::max<size_t>(1, atoms) * sizeof(int32_t));
    pb.frame_host.get(kFrameWords);
    pb.frame_read.prepare();
}

void prepare_frame(hipStream_t stream, PreparedBatch& pb) {
    const int64_t S = pb.structures, atoms = pb.atoms;
    pb.cells_total = pb.wave_cells = pb.big_bound = pb.chunks = pb.small_structs = pb.large_structs = 0;
    pb.direct_bins = pb.struct_bins = false;
    if (S == 0 || atoms == 0) return;
    char* base = static_cast<char*>(pb.d_frame.ptr);
    auto* box = reinterpret_cast<unsigned long long*>(base);
    auto* span = reinterpret_cast<uint32_t*>(base + pb.frame_span);
    auto* vol = reinterpret_cast<int64_t*>(base + pb.frame_vol);
    auto* cls = reinterpret_cast<int32_t*>(base + pb.frame_cls);
    auto* nch = reinterpret_cast<int32_t*>(base + pb.frame_nch);
    auto* summary = reinterpret_cast<unsigned long long*>(base + pb.frame_summary);
    StructGeom* geom = pb.d_geom.as<StructGeom>();
    const double* pos = pb.d_positions.as<double>();
    const int32_t* atom_struct = pb.d_atom_struct.as<int32_t>();
    MDX_HIP(hipMemsetAsync(pb.d_frame.ptr, 0, pb.frame_bytes, stream));
    hipLaunchKernelGGL(k_frame_bounds, dim3(frame_grid_size(atoms)), dim3(kFrameThreads), 0, stream, pos, atom_struct,
                       atoms, box, summary);
    hipLaunchKernelGGL(k_frame_span, dim3(frame_grid_size(atoms)), dim3(kFrameThreads), 0, stream, pos, atom_struct,
                       atoms, geom, box, pb.cutoff, span, pb.d_atom_cell.as<unsigned long long>());
    hipLaunchKernelGGL(k_frame_classify, dim3(frame_grid_size(S)), dim3(kFrameThreads), 0, stream, geom, S, box, span,
                       pb.cutoff, vol, cls, nch, summary);
    hipLaunchKernelGGL(k_frame_lists, dim3(1), dim3(kListThreads), 0, stream, geom, S, vol, cls, nch,
                       pb.d_struct_cells.as<int64_t>(), pb.d_cell_lists.as<int32_t>(), pb.d_struct_list.as<int32_t>(),
                       pb.d_bin_chunks.as<BinChunk>(), summary);
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
}

void place_centres(hipStream_t stream, const PreparedBatch& pb, DeviceGraph& gr, int32_t* centre_count) {
    const int64_t atoms = pb.atoms, cells = pb.cells_total;
    gr.cell_centre_start.reserve(static_cast<size_t>(cells + 1) * sizeof(int64_t));
    gr.cell_struct.reserve(std::max<size_t>(1, static_cast<size_t>(cells)) * sizeof(int32_t));
    if (atoms == 0 || cells == 0) return;
    char* base = static_cast<char*>(pb.d_frame.ptr);
    auto* summary = reinterpret_cast<unsigned long long*>(base + pb.frame_summary);
    hipLaunchKernelGGL(k_frame_homes, dim3(frame_grid_size(atoms)), dim3(kFrameThreads), 0, stream,
                       pb.d_atom_struct.as<int32_t>(), atoms, pb.d_geom.as<StructGeom>(),
                       pb.d_atom_cell.as<unsigned long long>(), centre_count, pb.d_atom_home.as<int32_t>(),
                       pb.d_atom_rank.as<int32_t>(), pb.d_cell_lists.as<int32_t>(), pb.wave_cells,
                       pb.structures + atoms, summary);
    scan_counts(stream, centre_count, gr.cell_centre_start.as<int64_t>(), cells, gr.scan_tmp);
    hipLaunchKernelGGL(k_frame_place, dim3(frame_grid_size(std::max(atoms, cells))), dim3(kFrameThreads), 0, stream,
                       atoms, pb.d_atom_home.as<int32_t>(), pb.d_atom_rank.as<int32_t>(),
                       gr.cell_centre_start.as<int64_t>(), pb.d_cell_centres.as<int32_t>(), cells,
                       pb.d_struct_cells.as<int64_t>(), pb.structures, gr.cell_struct.as<int32_t>());
    MDX_HIP(hipGetLastError());
}

} // namespace mdx
