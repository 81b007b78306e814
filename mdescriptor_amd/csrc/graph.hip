// Kernel 1: periodic / isolated cell-list neighbour search on gfx950.
//
// The pair set is the reference's (build_structure_graph, image-extended
// path, cpp/src/common/neighbor.cpp:423-679): every (atom j, image n) with
// n in [-b, b]^3 and |r_j + n.cell - r_i|^2 <= cutoff^2, self pair and
// self-images included, on raw (unwrapped) positions.  The cell grid is the
// reference's own (build_grid, neighbor.cpp:135-194: bounding box of all
// images, 1e-10 padding, cells at least `cutoff` wide), so each centre visits
// the same 27 cells in the same z/y/x order and finds candidates in the same
// order; rows therefore come out in the reference's order (grouped by
// neighbour species for SOAP, a stable partition of that order).
//
// Device pipeline (all on one stream):
//   bin_count -> scan -> bin_fill -> bin_sort   images into ROI cells, sorted
//   cell_species                                 first bin of each species per cell
//   centre_cell -> scan -> centre_fill           centres grouped by home cell
//   neighbors<count> -> scan of totals           per-centre, per-species counts
//   neighbors<fill>                              wave ballot compaction
// Only cells within one cell of some centre (the region of interest) are
// binned; the others are never visited.  The neighbour passes run one
// workgroup per home cell: its 27-cell candidate set is the same for every
// centre of the cell, so it is staged in LDS once and scanned by all of them.
#include "mdx_internal.h"

#include <type_traits>

#include <algorithm>
#include <chrono>
#include <thread>
#include <cmath>
#include <cstring>
#include <limits>
#include <unordered_map>

namespace mdx {

void check_hip(hipError_t code, const char* what) {
    if (code == hipSuccess) return;
    const char* name = hipGetErrorString(code);
    if (code == hipErrorOutOfMemory || code == hipErrorMemoryAllocation) {
        throw Error(MDX_OUT_OF_MEMORY, std::string("HIP out of memory in ") + what);
    }
    if (code == hipErrorNoDevice || code == hipErrorInvalidDevice || code == hipErrorInsufficientDriver) {
        throw Error(MDX_DEVICE_UNAVAILABLE, std::string("HIP device unavailable: ") + name);
    }
    throw Error(MDX_INTERNAL, std::string(what) + " failed: " + name);
}

void* ScratchArena::take(size_t size) {
    const size_t rounded = std::max<size_t>(256, (size + 255) & ~size_t(255));
    if (base == nullptr || rounded > capacity - used) {
        throw Error(MDX_INVALID_ARGUMENT, "the batch needs more device scratch than the static maximum of " +
                                              std::to_string(capacity) + " bytes");
    }
    void* p = base + used;
    used += rounded;
    return p;
}

void ScratchArena::rewind(void* piece) {
    char* p = static_cast<char*>(piece);
    if (p < base || p > base + used) throw Error(MDX_INTERNAL, "scratch piece outside its arena");
    used = static_cast<size_t>(p - base);
}

void DeviceBuffer::reserve(size_t size) {
    if (size <= bytes && ptr != nullptr) return;
    if (arena != nullptr) {
        ptr = arena->take(size);
        bytes = size;
        return;
    }
    release();
    const size_t rounded = std::max<size_t>(256, (size + 255) & ~size_t(255));
    MDX_HIP(hipMalloc(&ptr, rounded));
    bytes = rounded;
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

size_t device_workgroup_lds() {
    static int cached[64] = {};
    int dev = 0;
    MDX_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return 64 * 1024;
    if (cached[dev] == 0) {
        int bytes = 0;
        MDX_HIP(hipDeviceGetAttribute(&bytes, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
        cached[dev] = bytes > 0 ? bytes : 64 * 1024;
    }
    return static_cast<size_t>(cached[dev]);
}

PinnedWords::~PinnedWords() {
    if (words_ != nullptr) (void)hipHostFree(words_);
}

unsigned long long* PinnedWords::get(size_t count) {
    if (count > count_) {
        if (words_ != nullptr) MDX_HIP(hipHostFree(words_));
        words_ = nullptr;
        count_ = 0;
        void* p = nullptr;
        MDX_HIP(hipHostMalloc(&p, count * sizeof(unsigned long long), hipHostMallocDefault));
        words_ = static_cast<unsigned long long*>(p);
        count_ = count;
    }
    return words_;
}

StreamPoint::~StreamPoint() {
    if (event_ != nullptr) (void)hipEventDestroy(event_);
}

void StreamPoint::prepare() {
    if (event_ == nullptr) MDX_HIP(hipEventCreateWithFlags(&event_, hipEventDisableTiming));
}

void StreamPoint::wait(hipStream_t stream) {
    record(stream);
    sync();
}

void StreamPoint::record(hipStream_t stream) {
    prepare();
    MDX_HIP(hipEventRecord(event_, stream));
}

void StreamPoint::sync() {
    // Poll first: the short waits (the graph statistics) would otherwise pay
    // a blocking synchronisation's wake-up of tens of microseconds.  Past
    // 200 us of polling yield the core between polls, past 2 ms block.
    const auto start = std::chrono::steady_clock::now();
    for (;;) {
        const hipError_t e = hipEventQuery(event_);
        if (e == hipSuccess) return;
        if (e != hipErrorNotReady) MDX_HIP(e);
        const auto waited = std::chrono::steady_clock::now() - start;
        if (waited > std::chrono::milliseconds(2)) {
            MDX_HIP(hipEventSynchronize(event_));
            return;
        }
        if (waited > std::chrono::microseconds(200)) std::this_thread::yield();
    }
}

void DeviceBuffer::release() {
    if (ptr != nullptr && arena == nullptr) {
        (void)hipFree(ptr);
    }
    ptr = nullptr;
    bytes = 0;
}

namespace {

// ---------------------------------------------------------------- host side

double det3(const double* m) {
    return m[0] * (m[4] * m[8] - m[5] * m[7]) - m[1] * (m[3] * m[8] - m[5] * m[6])
        + m[2] * (m[3] * m[7] - m[4] * m[6]);
}

// inverse (math3.hpp:52-68), same cofactor order and division
bool inverse3(const double* m, double* r) {
    const double d = det3(m);
    if (!std::isfinite(d) || std::abs(d) < 1e-14) return false;
    r[0] = (m[4] * m[8] - m[5] * m[7]) / d;
    r[1] = (m[2] * m[7] - m[1] * m[8]) / d;
    r[2] = (m[1] * m[5] - m[2] * m[4]) / d;
    r[3] = (m[5] * m[6] - m[3] * m[8]) / d;
    r[4] = (m[0] * m[8] - m[2] * m[6]) / d;
    r[5] = (m[2] * m[3] - m[0] * m[5]) / d;
    r[6] = (m[3] * m[7] - m[4] * m[6]) / d;
    r[7] = (m[1] * m[6] - m[0] * m[7]) / d;
    r[8] = (m[0] * m[4] - m[1] * m[3]) / d;
    return true;
}

// validate_batch (cpp/include/mdescriptor/detail/batch.hpp:19-80)
void validate_batch(const mdx_batch_view& b) {
    if (b.structures < 0 || b.atoms < 0 || b.offsets == nullptr) {
        throw Error(MDX_INVALID_ARGUMENT, "invalid structure batch");
    }
    if (b.structures == 0) {
        if (b.atoms != 0 || b.offsets[0] != 0) {
            throw Error(MDX_INVALID_ARGUMENT, "empty structure batch has non-empty atom data");
        }
        return;
    }
    if (b.numbers == nullptr || b.positions == nullptr || b.cells == nullptr || b.pbc == nullptr) {
        throw Error(MDX_INVALID_ARGUMENT, "structure batch contains null arrays");
    }
    if (b.offsets[0] != 0 || b.offsets[b.structures] != b.atoms) {
        throw Error(MDX_INVALID_ARGUMENT, "offsets do not describe the flattened arrays");
    }
    for (int64_t s = 0; s < b.structures; ++s) {
        if (b.offsets[s] < 0 || b.offsets[s] > b.offsets[s + 1] || b.offsets[s + 1] > b.atoms) {
            throw Error(MDX_INVALID_ARGUMENT, "offsets must be monotonic");
        }
        bool periodic = true, isolated = true;
        for (int a = 0; a < 3; ++a) {
            const int32_t f = b.pbc[s * 3 + a];
            if (f != 0 && f != 1) throw Error(MDX_INVALID_ARGUMENT, "pbc must contain only 0 or 1");
            periodic = periodic && f == 1;
            isolated = isolated && f == 0;
        }
        if (!periodic && !isolated) {
            throw Error(MDX_INVALID_ARGUMENT, "mixed periodicity is not supported; use all-zero or all-one pbc");
        }
        const double* cell = b.cells + s * 9;
        for (int i = 0; i < 9; ++i) {
            if (!std::isfinite(cell[i])) throw Error(MDX_INVALID_ARGUMENT, "cells must be finite");
        }
        const double d = det3(cell);
        if (periodic && (!std::isfinite(d) || std::abs(d) < 1e-14)) {
            throw Error(MDX_INVALID_ARGUMENT, "cells must be nonsingular");
        }
    }
    for (int64_t i = 0; i < b.atoms; ++i) {
        if (b.numbers[i] <= 0) throw Error(MDX_INVALID_ARGUMENT, "atomic numbers must be positive");
        for (int a = 0; a < 3; ++a) {
            if (!std::isfinite(b.positions[i * 3 + a])) {
                throw Error(MDX_INVALID_ARGUMENT, "positions must be finite");
            }
        }
    }
}

// ---------------------------------------------------------------- device side

__device__ inline int64_t roi_cell(const StructGeom& g, double x, double y, double z, bool& inside) {
    const int cx = grid_coordinate(x, g.minimum[0], g.spacing[0], g.dims[0]);
    const int cy = grid_coordinate(y, g.minimum[1], g.spacing[1], g.dims[1]);
    const int cz = grid_coordinate(z, g.minimum[2], g.spacing[2], g.dims[2]);
    const int lx = cx - g.roi_lo[0], ly = cy - g.roi_lo[1], lz = cz - g.roi_lo[2];
    inside = lx >= 0 && ly >= 0 && lz >= 0 && lx < g.roi_dim[0] && ly < g.roi_dim[1] && lz < g.roi_dim[2];
    return g.cell_begin + lx + static_cast<int64_t>(g.roi_dim[0]) * (ly + static_cast<int64_t>(g.roi_dim[1]) * lz);
}

__device__ inline void image_position(const StructGeom& g, const ImageDesc* images, const double* positions,
                                      int64_t key, double& x, double& y, double& z, int64_t& atom,
                                      int64_t& image) {
    const int64_t q = key / g.natoms;
    const int64_t j = key - q * g.natoms;
    atom = g.atom_begin + j;
    image = g.image_begin + q;
    const ImageDesc& im = images[image];
    x = positions[atom * 3 + 0] + im.shift[0];
    y = positions[atom * 3 + 1] + im.shift[1];
    z = positions[atom * 3 + 2] + im.shift[2];
}

// Binning walks (image, atom) pairs on a 2-D grid (y: image, x: atom), so no
// index division is needed.  The extended index of (image q, local atom j) is

// q * natoms + j (neighbor.cpp:519-528).  Count pass: cell_count[c] += 1;
// fill pass: keys at cell_start[c] + a slot taken from cell_count.
template <bool kFill>
__global__ void k_bin_atoms(const StructGeom* geom, const ImageDesc* images, const double* positions,
                            const int32_t* atom_struct, const int32_t* types, int species_major, int64_t atoms,
                            int max_images, int32_t* cell_count, const int64_t* cell_start, uint64_t* keys) {
    for (int q = blockIdx.y; q < max_images; q += gridDim.y) {
        for (int64_t a = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; a < atoms;
             a += static_cast<int64_t>(gridDim.x) * blockDim.x) {
            const StructGeom& g = geom[atom_struct[a]];
            if (q >= g.n_images || g.lds_bins != 0) continue;
            const uint32_t j = static_cast<uint32_t>(a - g.atom_begin);
            const uint32_t ext = static_cast<uint32_t>(q) * static_cast<uint32_t>(g.natoms) + j;
            if (g.one_cell != 0) {
                // every image in the one cell: its count is known and the
                // extended index is a free slot (no atomics)
                const int64_t c = g.cell_begin;
                if (kFill) {
                    const uint64_t major = species_major ? static_cast<uint64_t>(types[a]) << 32 : 0;
                    keys[cell_start[c] + ext] = major | ext;
                } else if (ext == 0) {
                    cell_count[c] = g.natoms * g.n_images;
                }
                continue;
            }
            const ImageDesc& im = images[g.image_begin + q];
            bool inside;
            const int64_t c = roi_cell(g, positions[a * 3 + 0] + im.shift[0], positions[a * 3 + 1] + im.shift[1],
                                       positions[a * 3 + 2] + im.shift[2], inside);
            if (!inside) continue;
            if (kFill) {
                const int32_t slot = atomicAdd(&cell_count[c], 1);
                const uint64_t major = species_major ? static_cast<uint64_t>(types[a]) << 32 : 0;
                keys[cell_start[c] + slot] = major | ext;
            } else {
                atomicAdd(&cell_count[c], 1);
            }
        }
    }
}

// Binning of the structures with few ROI cells, a run of kBinChunk images
// per workgroup: each image takes a slot among the workgroup's images of its
// cell from an LDS counter; then one global atomic per (workgroup, cell)
// adds the workgroup's count (count pass) or reserves the workgroup's range
// of the cell (fill pass).  Same cells, keys and cell counts as
// k_bin_atoms; the order inside a cell is restored by k_bin_sort.
constexpr int kBinThreads = 512;
constexpr int kBinPer = kBinChunk / kBinThreads;

// The chunk of workgroup b: structure s is the last whose first chunk
// (struct_chunks, a scan of every structure's chunk count) is at or before
// b (structures without chunks share their successor's first chunk).
__device__ inline BinChunk bin_chunk(const int64_t* struct_chunks, int64_t structures, const StructGeom* geom,
                                     int64_t b) {
    int64_t lo = 0, hi = structures;
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) / 2;
        if (struct_chunks[mid] <= b) lo = mid; else hi = mid;
    }
    const int64_t first = (b - struct_chunks[lo]) * kBinChunk;
    const int64_t images = static_cast<int64_t>(geom[lo].natoms) * geom[lo].n_images;
    return BinChunk{first, static_cast<int32_t>(lo), static_cast<int32_t>(min<int64_t>(kBinChunk, images - first))};
}

template <bool kFill>
__global__ __launch_bounds__(kBinThreads) void k_bin_lds(const int64_t* struct_chunks, int64_t structures,
                                                         const StructGeom* geom,
                                                         const ImageDesc* images, const double* positions,
                                                         const int32_t* types, int species_major, int32_t* cell_count,
                                                         const int64_t* cell_start, uint64_t* keys) {
    __shared__ int32_t s_count[kLdsBinCells];
    __shared__ int32_t s_base[kFill ? kLdsBinCells : 1];
    const BinChunk ch = bin_chunk(struct_chunks, structures, geom, blockIdx.x);
    const StructGeom& g = geom[ch.structure];
    const int ncells = g.roi_dim[0] * g.roi_dim[1] * g.roi_dim[2];
    const int tid = threadIdx.x;
    for (int i = tid; i < ncells; i += kBinThreads) s_count[i] = 0;
    __syncthreads();
    int lc[kBinPer], slot[kBinPer];
#pragma unroll
    for (int r = 0; r < kBinPer; ++r) {
        const int e = tid + r * kBinThreads;
        lc[r] = -1;
        slot[r] = 0;
        if (e < ch.count) {
            const int64_t ext = ch.first + e;
            const int64_t q = ext / g.natoms;
            const int64_t a = g.atom_begin + (ext - q * g.natoms);
            const ImageDesc& im = images[g.image_begin + q];
            bool inside;
            const int64_t c = roi_cell(g, positions[a * 3 + 0] + im.shift[0], positions[a * 3 + 1] + im.shift[1],
                                       positions[a * 3 + 2] + im.shift[2], inside);
            if (inside) {
                lc[r] = static_cast<int>(c - g.cell_begin);
                slot[r] = atomicAdd(&s_count[lc[r]], 1);
            }
        }
    }
    __syncthreads();
    for (int i = tid; i < ncells; i += kBinThreads) {
        const int n = s_count[i];
        if (n == 0) continue;
        const int base = atomicAdd(&cell_count[g.cell_begin + i], n);
        if (kFill) s_base[i] = base;
    }
    if (!kFill) return;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kBinPer; ++r) {
        if (lc[r] < 0) continue;
        const int64_t ext = ch.first + tid + r * kBinThreads;
        const int64_t a = g.atom_begin + ext % g.natoms;
        const uint64_t major = species_major ? static_cast<uint64_t>(types[a]) << 32 : 0;
        const int64_t c = g.cell_begin + lc[r];
        keys[cell_start[c] + s_base[lc[r]] + slot[r]] = major | static_cast<uint64_t>(ext);
    }
}

// Order each cell by extended index (the reference fills cells in extended
// order, neighbor.cpp:184-192) -- species first in Bins mode -- by ranking,
// then materialise the binned images as SoA.  Keys are unique inside a cell.
__global__ void k_bin_sort(const StructGeom* geom, const int32_t* cell_struct, const ImageDesc* images,
                           const double* positions, const int32_t* types, const int64_t* cell_start,
                           int64_t cells_total, const uint64_t* keys, double* bx, double* by, double* bz,
                           int32_t* batom, int32_t* bimage, int32_t* btype, unsigned long long* stats) {
    // the binned image total, read back with the search statistics
    if (blockIdx.x == 0 && threadIdx.x == 0) stats[kStatBinned] = static_cast<unsigned long long>(cell_start[cells_total]);
    for (int64_t c = blockIdx.x; c < cells_total; c += gridDim.x) {
        const int64_t start = cell_start[c];
        const int64_t n = cell_start[c + 1] - start;
        if (n == 0) continue;
        const StructGeom& g = geom[cell_struct[c]];
        for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
            const uint64_t full = keys[start + i];
            int64_t rank = 0;
            for (int64_t j = 0; j < n; ++j) rank += keys[start + j] < full ? 1 : 0;
            const int64_t dest = start + rank;
            const int64_t key = static_cast<int64_t>(static_cast<uint32_t>(full));
            double x, y, z;
            int64_t atom, image;
            image_position(g, images, positions, key, x, y, z, atom, image);
            bx[dest] = x;
            by[dest] = y;
            bz[dest] = z;
            batom[dest] = static_cast<int32_t>(atom);
            bimage[dest] = static_cast<int32_t>(image);
            btype[dest] = types[atom];
        }
    }
}

// The runs of each cell: species t of cell c spans [runs[c*(S+1) + t],
// runs[c*(S+1) + t + 1]) (Bins mode: cells are sorted by species) and
// runs[c*(S+1) + S] is the cell's end.  One thread per (cell, t): a
// lower-bound search for t in the cell's sorted species column.
__global__ void k_cell_species(const int64_t* cell_start, int64_t cells_total, const int32_t* btype, int S,
                               int64_t* cell_runs) {
    const int64_t work = cells_total * (S + 1);
    for (int64_t w = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; w < work;
         w += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t c = w / (S + 1);
        const int t = static_cast<int>(w - c * (S + 1));
        int64_t lo = cell_start[c], hi = cell_start[c + 1];
        if (t == S) {
            lo = hi;
        } else if (S > 1) {
            while (lo < hi) {
                const int64_t mid = lo + (hi - lo) / 2;
                if (btype[mid] < t) lo = mid + 1; else hi = mid;
            }
        }
        cell_runs[w] = lo;
    }
}

// Binning of a whole structure by one workgroup, for batches whose every
// structure has at most kLdsBinCells ROI cells and kStructImages images:
// the image count of each cell in LDS, their scan, 32-bit keys (species
// << 16 | extended index) at the cells' places in LDS, the rank of each key
// inside its cell, then the binned images as SoA and each cell's runs.
// The structure's bins start at its first extended index (ext_begin), so no
// scan across structures is needed (the bins between its last binned image
// and the next structure's first stay unused).  Same cells, order and runs
// as k_bin_lds / k_bin_atoms + k_bin_sort + k_cell_species.
constexpr int kStructThreads = 1024;
constexpr int kStructPer = kStructImages / kStructThreads;
static_assert(kStructImages <= (1 << 16), "extended index below the species bits of a key");
constexpr int kStructCellsPer = kLdsBinCells / kStructThreads;

__global__ __launch_bounds__(kStructThreads) void k_bin_struct(const int32_t* list, const StructGeom* geom,
                                                               const ImageDesc* images, const double* positions,
                                                               const int32_t* types, int S, double* bx, double* by,
                                                               double* bz, int32_t* batom, int32_t* bimage,
                                                               int32_t* btype, int64_t* cell_runs,
                                                               unsigned long long* stats) {
    __shared__ int32_t s_count[kLdsBinCells];
    __shared__ int32_t s_start[kLdsBinCells];
    __shared__ uint32_t s_key[kStructImages];
    __shared__ int32_t s_wave[kStructThreads / kWave];
    const StructGeom& g = geom[list[blockIdx.x]];
    const int natoms = g.natoms;
    if (natoms == 0) return; // no cells
    const int ncells = g.roi_dim[0] * g.roi_dim[1] * g.roi_dim[2];
    const int n_ext = natoms * g.n_images;
    const int tid = threadIdx.x;
    const int lane = tid % kWave;
    const int wave = tid / kWave;
    for (int i = tid; i < ncells; i += kStructThreads) s_count[i] = 0;
    __syncthreads();
    // each image's ROI cell (every image of a one-cell structure is in its
    // one cell; -1: outside the region), all gathers first, then its slot
    // among the cell's images
    int lc[kStructPer], slot[kStructPer];
#pragma unroll
    for (int r = 0; r < kStructPer; ++r) {
        const int e = tid + r * kStructThreads;
        lc[r] = -1;
        if (e < n_ext) {
            int c = 0;
            bool inside = true;
            if (g.one_cell == 0) {
                const int q = e / natoms;
                const int64_t a = g.atom_begin + (e - q * natoms);
                const ImageDesc& im = images[g.image_begin + q];
                c = static_cast<int>(roi_cell(g, positions[a * 3 + 0] + im.shift[0],
                                              positions[a * 3 + 1] + im.shift[1],
                                              positions[a * 3 + 2] + im.shift[2], inside) - g.cell_begin);
            }
            if (inside) lc[r] = c;
        }
    }
#pragma unroll
    for (int r = 0; r < kStructPer; ++r) slot[r] = lc[r] >= 0 ? atomicAdd(&s_count[lc[r]], 1) : 0;
    __syncthreads();
    // exclusive scan of the cell counts, kStructCellsPer consecutive cells a thread
    int v[kStructCellsPer];
    int sum = 0;
#pragma unroll
    for (int k = 0; k < kStructCellsPer; ++k) {
        const int i = tid * kStructCellsPer + k;
        v[k] = i < ncells ? s_count[i] : 0;
        sum += v[k];
    }
    int incl = sum;
#pragma unroll
    for (int off = 1; off < kWave; off *= 2) {
        const int u = __shfl_up(incl, off);
        if (lane >= off) incl += u;
    }
    if (lane == kWave - 1) s_wave[wave] = incl;
    __syncthreads();
    int before = 0, binned = 0;
    for (int w = 0; w < kStructThreads / kWave; ++w) {
        if (w < wave) before += s_wave[w];
        binned += s_wave[w];
    }
    int run = before + incl - sum;
#pragma unroll
    for (int k = 0; k < kStructCellsPer; ++k) {
        const int i = tid * kStructCellsPer + k;
        if (i < ncells) s_start[i] = run;
        run += v[k];
    }
    __syncthreads();
    // keys at their cells' places, in slot order
    uint32_t key[kStructPer];
#pragma unroll
    for (int r = 0; r < kStructPer; ++r) {
        key[r] = 0;
        if (lc[r] < 0) continue;
        const int e = tid + r * kStructThreads;
        const int64_t a = g.atom_begin + e % natoms;
        key[r] = (S > 1 ? static_cast<uint32_t>(types[a]) << 16 : 0u) | static_cast<uint32_t>(e);
        s_key[s_start[lc[r]] + slot[r]] = key[r];
    }
    __syncthreads();
    // each image at its rank inside its cell: (species, extended index)
    // order; all ranks first, then the gathers and stores
    const int64_t base = g.ext_begin;
    int rank[kStructPer];
#pragma unroll
    for (int r = 0; r < kStructPer; ++r) {
        rank[r] = 0;
        if (lc[r] < 0) continue;
        const int st = s_start[lc[r]], n = s_count[lc[r]];
        int below = 0;
        for (int j = 0; j < n; ++j) below += s_key[st + j] < key[r] ? 1 : 0;
        rank[r] = st + below;
    }
#pragma unroll
    for (int r = 0; r < kStructPer; ++r) {
        if (lc[r] < 0) continue;
        const int64_t dest = base + rank[r];
        const int e = tid + r * kStructThreads;
        double x, y, z;
        int64_t atom, image;
        image_position(g, images, positions, e, x, y, z, atom, image);
        bx[dest] = x;
        by[dest] = y;
        bz[dest] = z;
        batom[dest] = static_cast<int32_t>(atom);
        bimage[dest] = static_cast<int32_t>(image);
        btype[dest] = types[atom];
    }
    // runs: the cell's keys below species t, and its end
    for (int w = tid; w < ncells * (S + 1); w += kStructThreads) {
        const int c = w / (S + 1), t = w - c * (S + 1);
        const int st = s_start[c], n = s_count[c];
        int below = n;
        if (t < S) {
            below = 0;
            for (int j = 0; j < n; ++j) below += static_cast<int>(s_key[st + j] >> 16) < t ? 1 : 0;
        }
        cell_runs[(g.cell_begin + c) * (S + 1) + t] = base + st + below;
    }
    // the binned image total, read back with the search statistics
    if (tid == 0 && binned > 0) {
        atomicAdd(&stats[stat_binned(static_cast<int>(blockIdx.x % kStatLanes))], static_cast<unsigned long long>(binned));
    }
}

// Binning of structures of at most a wavefront of images and kSmallCells ROI
// cells (small molecules), a wavefront each: lane e holds image e and its
// key (ROI cell << 11 | species << 6 | e; images outside the region sort
// last); its rank among the structure's keys is its bin, from the
// structure's first extended index as in k_bin_struct, and the runs of a
// cell count the keys below (cell, species t) for t = 0 .. S (t = S: the
// cell's end).  Same cells, order and runs as the other binning paths.
static_assert(kMaxSpecies < 32 && kSmallImages <= 64, "species and image fields of a small structure's key");

__global__ __launch_bounds__(kBlock) void k_bin_small(const int32_t* list, int64_t count, const StructGeom* geom,
                                                      const ImageDesc* images, const double* positions,
                                                      const int32_t* types, int S, double* bx, double* by, double* bz,
                                                      int32_t* batom, int32_t* bimage, int32_t* btype,
                                                      int64_t* cell_runs, unsigned long long* stats) {
    constexpr int kWaves = kBlock / kWave;
    const int lane = threadIdx.x % kWave;
    const int64_t w = static_cast<int64_t>(blockIdx.x) * kWaves + threadIdx.x / kWave;
    if (w >= count) return;
    const StructGeom& g = geom[list[w]];
    const int n_ext = g.natoms * g.n_images; // at most kSmallImages (the host's choice)
    const int ncells = g.roi_dim[0] * g.roi_dim[1] * g.roi_dim[2];
    constexpr uint32_t kOutside = 0xffffffffu;
    uint32_t key = kOutside;
    double x = 0.0, y = 0.0, z = 0.0;
    int64_t atom = 0, image = 0;
    if (lane < n_ext) {
        image_position(g, images, positions, lane, x, y, z, atom, image);
        int c = 0;
        bool inside = true;
        if (g.one_cell == 0) c = static_cast<int>(roi_cell(g, x, y, z, inside) - g.cell_begin);
        if (inside) {
            key = (static_cast<uint32_t>(c) << 11) | (static_cast<uint32_t>(types[atom]) << 6) |
                  static_cast<uint32_t>(lane);
        }
    }
    int rank = 0;
    for (int j = 0; j < n_ext; ++j) {
        rank += static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(key), j)) < key ? 1 : 0;
    }
    const int64_t base = g.ext_begin;
    if (key != kOutside) {
        const int64_t dest = base + rank;
        bx[dest] = x;
        by[dest] = y;
        bz[dest] = z;
        batom[dest] = static_cast<int32_t>(atom);
        bimage[dest] = static_cast<int32_t>(image);
        btype[dest] = types[atom];
    }
    const int pairs = ncells * (S + 1);
    for (int p0 = 0; p0 < pairs; p0 += kWave) {
        const int p = p0 + lane;
        const int c = p / (S + 1), t = p - c * (S + 1);
        const uint32_t bound = (static_cast<uint32_t>(c) << 11) | (static_cast<uint32_t>(t) << 6);
        int below = 0;
        for (int j = 0; j < n_ext; ++j) {
            below += static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(key), j)) < bound ? 1 : 0;
        }
        if (p < pairs) cell_runs[(g.cell_begin + c) * (S + 1) + t] = base + below;
    }
    const int binned = static_cast<int>(__popcll(__ballot(key != kOutside)));
    if (lane == 0 && binned > 0) {
        atomicAdd(&stats[stat_binned(static_cast<int>(w % kStatLanes))], static_cast<unsigned long long>(binned));
    }
}

// Kernel 1: the neighbour rows of the centres of one home cell per
// workgroup.  The 27 cells around the home cell are visited in the
// reference's order (z outer, y, x inner, cells outside the grid skipped;
// neighbor.cpp:558-566) and the binned images of a cell in extended order.
// With several species the bins of a cell are sorted by species first and
// the walk is species-major (species, then the 27 cells), so a centre's rows
// come out grouped by species and, inside a species, in the reference's
// candidate order; with one species they are exactly the reference's rows.
// That candidate sequence is the same for every centre of the cell: the
// workgroup stages it in LDS (kStage candidates at a time) and each
// wavefront scans it for one centre after another.  Count pass
// (kNbrCount): per-species counts and row totals.  Fill pass (kNbrFill): the
// bin index of every accepted image at pair_start[centre] onwards (wave
// ballot + popcount compaction).  Slotted pass (kNbrSlotted, the SOAP
// expansion's layout): both at once, each centre's rows at centre * cap
// onwards (rows past cap are dropped; the statistics lines receive the total
// rows).  Both counting passes record the largest row count of a centre there.
constexpr int kNbrThreads = 512;
constexpr int kNbrWaves = kNbrThreads / kWave;
constexpr int kStage = 1024;        // candidates staged in LDS per pass over a cell's centres
constexpr int kCentreBatch = 128;   // centres whose running counts live in LDS at once
constexpr int kSegments = kMaxSpecies * 27;
constexpr int kNoBoundary = 0x7fffffff;
constexpr int kNbrCount = 0, kNbrFill = 1, kNbrSlotted = 2;

// a wave-uniform 64-bit value in scalar registers
__device__ inline int64_t uniform_i64(int64_t v) {
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v >> 32)));
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ inline uint64_t lane_range(int lo, int hi) {
    // bits lo .. hi-1 of a 64-lane mask, 0 <= lo <= hi <= 64
    const uint64_t upto_hi = hi >= 64 ? ~0ull : ((1ull << hi) - 1ull);
    const uint64_t upto_lo = lo >= 64 ? ~0ull : ((1ull << lo) - 1ull);
    return upto_hi & ~upto_lo;
}

template <int kMode>
__global__ __launch_bounds__(kNbrThreads) void k_neighbors(
    const StructGeom* geom, const int32_t* cell_struct, const double* positions, const int32_t* cell_list,
    const unsigned long long* list_count, const int64_t* cell_centre_start, const int32_t* cell_centres, const int64_t* cell_runs,
    const double* bx, const double* by, const double* bz, int S,
    double accept_max, int32_t* counts, int32_t* totals, int64_t* pair_start, uint32_t* pair_bin, int64_t cap,
    unsigned long long* stats) {
    constexpr bool kFill = kMode == kNbrFill;
    constexpr bool kCount = kMode != kNbrFill;
    constexpr bool kWrite = kMode != kNbrCount;
    __shared__ double2 s_xy[kStage];          // candidate x, y
    __shared__ double2 s_zb[kStage];          // candidate z, bin index (bit pattern)
    __shared__ int64_t s_segstart[kSegments]; // first bin of segment (species, cell k)
    __shared__ int32_t s_segpre[kSegments + 1];
    __shared__ int32_t s_centre[kCentreBatch];
    __shared__ double s_cpos[kCentreBatch * 3]; // centre positions of the batch
    __shared__ int64_t s_first[kCentreBatch];   // first output row of each centre (fill pass)
    __shared__ int32_t s_found[kCentreBatch];
    __shared__ int32_t s_limit[kCentreBatch];   // rows of each centre (fill pass)
    // rows of a centre before species boundary t (count pass)
    __shared__ int32_t s_bfound[kCentreBatch * kMaxSpecies];
    const int tid = threadIdx.x;
    const int lane = tid % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int nseg = S * 27;
    // the cells of the list
    const int64_t listed = static_cast<int64_t>(*list_count);
    for (int64_t w = blockIdx.x; w < listed; w += gridDim.x) {
        const int64_t c = static_cast<int64_t>(cell_list[w]);
        const int64_t c0 = cell_centre_start[c], c1 = cell_centre_start[c + 1];
        if (c0 == c1) continue;
        const StructGeom& g = geom[cell_struct[c]];
        // segments in walk order: index sp * 27 + k, k = the z/y/x cell offset
        for (int t = tid; t < nseg; t += kNbrThreads) {
            const int sp = t / 27, k = t - sp * 27;
            const int64_t local = c - g.cell_begin;
            const int ix = g.roi_lo[0] + static_cast<int>(local % g.roi_dim[0]) + k % 3 - 1;
            const int iy = g.roi_lo[1] + static_cast<int>((local / g.roi_dim[0]) % g.roi_dim[1]) + (k / 3) % 3 - 1;
            const int iz = g.roi_lo[2] + static_cast<int>(local / (static_cast<int64_t>(g.roi_dim[0]) * g.roi_dim[1]))
                + k / 9 - 1;
            int64_t start = 0, len = 0;
            if (ix >= 0 && iy >= 0 && iz >= 0 && ix < g.dims[0] && iy < g.dims[1] && iz < g.dims[2]) {
                const int64_t nc = g.cell_begin + (ix - g.roi_lo[0])
                    + static_cast<int64_t>(g.roi_dim[0])
                        * ((iy - g.roi_lo[1]) + static_cast<int64_t>(g.roi_dim[1]) * (iz - g.roi_lo[2]));
                start = cell_runs[nc * (S + 1) + sp];
                const int64_t end = cell_runs[nc * (S + 1) + sp + 1];
                len = end - start;
            }
            s_segstart[t] = start;
            s_segpre[t + 1] = static_cast<int32_t>(len);
        }
        __syncthreads();
        if (wave == 0) {
            // inclusive scan of the segment lengths, 64 at a time
            int32_t carry = 0;
            for (int t0 = 0; t0 < nseg; t0 += kWave) {
                const int t = t0 + lane;
                int32_t v = t < nseg ? s_segpre[t + 1] : 0;
#pragma unroll
                for (int off = 1; off < kWave; off *= 2) {
                    const int32_t u = __shfl_up(v, off);
                    if (lane >= off) v += u;
                }
                if (t < nseg) s_segpre[t + 1] = carry + v;
                carry += __shfl(v, kWave - 1);
            }
            if (lane == 0) s_segpre[0] = 0;
        }
        __syncthreads();
        const int total = s_segpre[nseg];
        for (int64_t b0 = c0; b0 < c1; b0 += kCentreBatch) {
            const int nb = static_cast<int>(min<int64_t>(kCentreBatch, c1 - b0));
            for (int i = tid; i < nb; i += kNbrThreads) {
                const int32_t centre = cell_centres[b0 + i];
                s_centre[i] = centre;
                s_cpos[i * 3 + 0] = positions[static_cast<int64_t>(centre) * 3 + 0];
                s_cpos[i * 3 + 1] = positions[static_cast<int64_t>(centre) * 3 + 1];
                s_cpos[i * 3 + 2] = positions[static_cast<int64_t>(centre) * 3 + 2];
                s_first[i] = kFill ? pair_start[centre] : kMode == kNbrSlotted ? centre * cap : 0;
                if (kFill) s_limit[i] = totals[centre];
                s_found[i] = 0;
            }
            for (int i = tid; i < nb * S; i += kNbrThreads) s_bfound[i] = 0;
            __syncthreads();
            for (int v0 = 0; v0 < total; v0 += kStage) {
                const int len = min(kStage, total - v0);
                const int glen = (len + kWave - 1) / kWave * kWave;
                // each thread stages up to kStage / kNbrThreads candidates, all
                // bin lookups first so that their global loads are in flight together
                constexpr int kPer = kStage / kNbrThreads;
                int64_t bins[kPer];
#pragma unroll
                for (int r = 0; r < kPer; ++r) {
                    const int i = tid + r * kNbrThreads;
                    const int v = v0 + min(i, len - 1);
                    // last segment starting at or before v (empty segments repeat a start)
                    int lo = 0, hi = nseg;
                    while (hi - lo > 1) {
                        const int mid = (lo + hi) / 2;
                        if (s_segpre[mid] <= v) lo = mid; else hi = mid;
                    }
                    bins[r] = s_segstart[lo] + (v - s_segpre[lo]);
                }
                double cx[kPer], cy[kPer], cz[kPer];
#pragma unroll
                for (int r = 0; r < kPer; ++r) {
                    cx[r] = bx[bins[r]];
                    cy[r] = by[bins[r]];
                    cz[r] = bz[bins[r]];
                }
#pragma unroll
                for (int r = 0; r < kPer; ++r) {
                    const int i = tid + r * kNbrThreads;
                    if (i < len) {
                        s_xy[i] = make_double2(cx[r], cy[r]);
                        s_zb[i] = make_double2(cz[r], __longlong_as_double(bins[r]));
                    } else if (i < glen) {
                        // pad to whole wavefronts with candidates at infinity (d^2 = inf)
                        s_xy[i] = make_double2(__builtin_huge_val(), 0.0);
                        s_zb[i] = make_double2(0.0, 0.0);
                    }
                }
                __syncthreads();
                for (int ci = wave; ci < nb; ci += kNbrWaves) {
                    const double px = s_cpos[ci * 3 + 0];
                    const double py = s_cpos[ci * 3 + 1];
                    const double pz = s_cpos[ci * 3 + 2];
                    int32_t found = s_found[ci];
                    // the centre's rows: from its first row, at most its counted
                    // total (fill) or the slot capacity (slotted)
                    const int64_t first_row = kWrite ? uniform_i64(s_first[ci]) : 0;
                    const int64_t limit = kFill ? s_limit[ci] : kWrite ? cap : 0;
                    const __amdgpu_buffer_rsrc_t rows = __builtin_amdgcn_make_buffer_rsrc(
                        pair_bin + first_row, 0, static_cast<int>(limit * sizeof(uint32_t)), 0x00020000);
                    // next species boundary of the walk at or after v0 (count pass)
                    int t_next = 1;
                    int bnext = kNoBoundary;
                    if (kCount) {
                        while (t_next < S && __builtin_amdgcn_readfirstlane(s_segpre[t_next * 27]) < v0) ++t_next;
                        bnext = t_next < S ? __builtin_amdgcn_readfirstlane(s_segpre[t_next * 27]) : kNoBoundary;
                    }
                    // bookkeeping of one wavefront-wide group of candidates at i0
                    auto account = [&](int i0, bool accept, uint64_t mask, uint32_t b) {
                        if (kWrite && accept) {
                            // row = rows so far + accepted lanes below this one; the
                            // descriptor's range drops rows past the slot capacity
                            const uint32_t row = __builtin_amdgcn_mbcnt_hi(
                                static_cast<uint32_t>(mask >> 32),
                                __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), static_cast<uint32_t>(found)));
                            __builtin_amdgcn_raw_buffer_store_b32(b, rows, static_cast<int>(row * sizeof(uint32_t)), 0, 0);
                        }
                        if (kCount) {
                            while (bnext < v0 + i0 + kWave) {
                                // rows before the boundary: earlier groups plus this group's lanes below it
                                const int k = bnext - (v0 + i0);
                                if (lane == 0) {
                                    s_bfound[ci * S + t_next] =
                                        found + static_cast<int32_t>(__popcll(mask & lane_range(0, k)));
                                }
                                ++t_next;
                                bnext = t_next < S ? __builtin_amdgcn_readfirstlane(s_segpre[t_next * 27]) : kNoBoundary;
                            }
                        }
                        found += static_cast<int32_t>(__popcll(mask));
                    };
                    // displacement = image - centre; d^2 = (dx*dx + dy*dy) + dz*dz
                    // (neighbor.cpp:569, math3.hpp:31-35), no contraction; accepted
                    // when d^2 <= accept_max (the host folds the boundary rule into it)
                    auto test = [&](int i, bool& accept, uint32_t& b) {
                        const double2 xy = s_xy[i];
                        const double2 zb = s_zb[i];
                        const double dx = xy.x - px;
                        const double dy = xy.y - py;
                        const double dz = zb.x - pz;
                        const double d2 = dx * dx + dy * dy + dz * dz;
                        accept = d2 <= accept_max;
                        b = static_cast<uint32_t>(__double_as_longlong(zb.y));
                    };
                    int i0 = 0;
                    // four groups per iteration: their LDS reads are in
                    // flight together (two: config 2's search 4 % slower)
                    for (; i0 + 4 * kWave <= glen; i0 += 4 * kWave) {
                        bool a0, a1, a2, a3;
                        uint32_t b0, b1, b2, b3;
                        test(i0 + lane, a0, b0);
                        test(i0 + kWave + lane, a1, b1);
                        test(i0 + 2 * kWave + lane, a2, b2);
                        test(i0 + 3 * kWave + lane, a3, b3);
                        const uint64_t m0 = __ballot(a0);
                        const uint64_t m1 = __ballot(a1);
                        const uint64_t m2 = __ballot(a2);
                        const uint64_t m3 = __ballot(a3);
                        account(i0, a0, m0, b0);
                        account(i0 + kWave, a1, m1, b1);
                        account(i0 + 2 * kWave, a2, m2, b2);
                        account(i0 + 3 * kWave, a3, m3, b3);
                    }
                    for (; i0 < glen; i0 += kWave) {
                        bool a0;
                        uint32_t b0;
                        test(i0 + lane, a0, b0);
                        account(i0, a0, __ballot(a0), b0);
                    }
                    if (lane == 0) s_found[ci] = found;
                }
                __syncthreads();
            }
            if (kCount) {
                if (tid == 0) {
                    atomicAdd(&stats[stat_centres(static_cast<int>(blockIdx.x % kStatLanes))],
                              static_cast<unsigned long long>(nb));
                }
                for (int i = tid; i < nb; i += kNbrThreads) {
                    totals[s_centre[i]] = s_found[i];
                    const int sl = static_cast<int>((blockIdx.x + static_cast<unsigned>(i)) % kStatLanes);
                    atomicMax(&stats[stat_most(sl)], static_cast<unsigned long long>(s_found[i]));
                    if (kMode == kNbrSlotted) {
                        pair_start[s_centre[i]] = s_first[i];
                        atomicAdd(&stats[stat_rows(sl)], static_cast<unsigned long long>(s_found[i]));
                    }
                }
                for (int i = tid; i < nb * S; i += kNbrThreads) {
                    const int ci = i / S, t = i - ci * S;
                    // rows before boundaries t and t + 1 (boundary 0 is the start; a
                    // boundary at or past the end of the walk is the centre's total)
                    int32_t lo = t == 0 ? 0 : s_segpre[t * 27] >= total ? s_found[ci] : s_bfound[i];
                    int32_t hi = t + 1 == S || s_segpre[(t + 1) * 27] >= total ? s_found[ci] : s_bfound[i + 1];
                    if (kMode == kNbrSlotted) {
                        // an overflowing centre's counts cover only the rows its
                        // slot holds, so a consumer launched before the host sees
                        // the overflow reads no row past the slot (the totals and
                        // the statistics keep the true counts)
                        lo = static_cast<int32_t>(min<int64_t>(lo, cap));
                        hi = static_cast<int32_t>(min<int64_t>(hi, cap));
                    }
                    counts[static_cast<int64_t>(s_centre[ci]) * S + t] = hi - lo;
                }
            }
            __syncthreads();
        }
    }
}

// Kernel 1 for the cells of structures whose region of interest is a single
// cell holding at most one wavefront of binned images (small molecules):
// every image of the structure is a candidate of each of its centres, and
// the 27-cell walk of k_neighbors visits only the home cell, so its candidate
// sequence is the cell's bins in order.  One wavefront per cell, candidate =
// lane: per centre one distance test, a ballot, and the rows written at
// their place in the sequence (mbcnt); the counts per species are the
// ballot's popcounts over the species' lane ranges.  Same passes, rows and
// counts as k_neighbors.
template <int kMode>
__global__ __launch_bounds__(kBlock) void k_neighbors_wave(
    const int32_t* wave_cells, int64_t n_cells, const double* positions, const int64_t* cell_centre_start,
    const int32_t* cell_centres, const int64_t* cell_runs, const double* bx,
    const double* by, const double* bz, int S, double accept_max, int32_t* counts, int32_t* totals,
    int64_t* pair_start, uint32_t* pair_bin, int64_t cap, unsigned long long* stats) {
    constexpr bool kFill = kMode == kNbrFill;
    constexpr bool kCount = kMode != kNbrFill;
    constexpr bool kWrite = kMode != kNbrCount;
    constexpr int kWavesPerBlock = kBlock / kWave;
    const int lane = threadIdx.x % kWave;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
    int32_t most = 0;
    int64_t rows_total = 0;
    int64_t searched = 0; // centres
    for (int64_t w = uniform_i64(static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave);
         w < n_cells; w += stride) {
        const int64_t c = uniform_i64(wave_cells[w]);
        const int64_t start = uniform_i64(cell_runs[c * (S + 1)]);
        // at most a wavefront of images (the host's choice of these cells)
        const int n = __builtin_amdgcn_readfirstlane(
            static_cast<int>(min<int64_t>(cell_runs[c * (S + 1) + S] - start, kWave)));
        if (n <= 0) continue;
        const bool real = lane < n;
        const uint32_t bin = static_cast<uint32_t>(start + (real ? lane : 0));
        const double x = bx[bin], y = by[bin], z = bz[bin];
        // species t of the cell at lanes [lo, hi) (lane t holds its own range)
        int lo = 0, hi = n;
        if (kCount && S > 1 && lane < S) {
            lo = static_cast<int>(cell_runs[c * (S + 1) + lane] - start);
            hi = min(n, static_cast<int>(cell_runs[c * (S + 1) + lane + 1] - start));
        }
        const uint64_t species_lanes = lane_range(lo, hi);
        // the cell's centres (the structure's atoms, at most a wavefront) one
        // per lane, read into scalars centre by centre
        const int64_t k0 = uniform_i64(cell_centre_start[c]);
        const int nk = __builtin_amdgcn_readfirstlane(
            static_cast<int>(min<int64_t>(uniform_i64(cell_centre_start[c + 1]) - k0, kWave)));
        if (nk <= 0) continue;
        const int my_centre = cell_centres[k0 + min(lane, nk - 1)];
        const double cx = positions[static_cast<int64_t>(my_centre) * 3 + 0];
        const double cy = positions[static_cast<int64_t>(my_centre) * 3 + 1];
        const double cz = positions[static_cast<int64_t>(my_centre) * 3 + 2];
        for (int k = 0; k < nk; ++k) {
            const int64_t centre = __builtin_amdgcn_readlane(my_centre, k);
            const double px = __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(cx), k),
                                               __builtin_amdgcn_readlane(__double2loint(cx), k));
            const double py = __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(cy), k),
                                               __builtin_amdgcn_readlane(__double2loint(cy), k));
            const double pz = __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(cz), k),
                                               __builtin_amdgcn_readlane(__double2loint(cz), k));
            // displacement = image - centre; d^2 = (dx*dx + dy*dy) + dz*dz, no
            // contraction (as k_neighbors)
            const double dx = x - px;
            const double dy = y - py;
            const double dz = z - pz;
            const double d2 = dx * dx + dy * dy + dz * dz;
            const bool accept = real && d2 <= accept_max;
            const uint64_t mask = __ballot(accept);
            const int32_t found = static_cast<int32_t>(__popcll(mask));
            if (kWrite) {
                const int64_t first = kFill ? uniform_i64(pair_start[centre]) : centre * cap;
                const int64_t limit = kFill ? static_cast<int64_t>(totals[centre]) : cap;
                const uint32_t row = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                                               __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
                if (accept && row < limit) pair_bin[first + row] = bin;
            }
            if (kCount) {
                if (lane < S) counts[centre * S + lane] = static_cast<int32_t>(__popcll(mask & species_lanes));
                if (lane == 0) {
                    totals[centre] = found;
                    if (kMode == kNbrSlotted) pair_start[centre] = centre * cap;
                }
                most = max(most, found);
                rows_total += found;
            }
        }
        searched += nk;
    }
    if (kCount && lane == 0) {
        const int sl = static_cast<int>((blockIdx.x * kWavesPerBlock + threadIdx.x / kWave) % kStatLanes);
        if (searched > 0) atomicAdd(&stats[stat_centres(sl)], static_cast<unsigned long long>(searched));
        if (most > 0) atomicMax(&stats[stat_most(sl)], static_cast<unsigned long long>(most));
        if (kMode == kNbrSlotted && rows_total > 0) {
            atomicAdd(&stats[stat_rows(sl)], static_cast<unsigned long long>(rows_total));
        }
    }
}

// ------------------------------------------------------------------ scan
constexpr int kScanItems = 8;
constexpr int kScanTile = kBlock * kScanItems;

// Exclusive scan over the workgroup (kThreads threads): wavefront scans by
// shuffles, then the wavefront totals through LDS (lds holds at least
// kThreads / kWave values).
template <int kThreads = kBlock>
__device__ int64_t block_exclusive_scan(int64_t value, int64_t* lds, int64_t& total) {
    constexpr int kWaves = kThreads / kWave;
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    int64_t inclusive = value;
#pragma unroll
    for (int offset = 1; offset < kWave; offset *= 2) {
        const int64_t add = __shfl_up(inclusive, offset);
        if (lane >= offset) inclusive += add;
    }
    if (lane == kWave - 1) lds[wave] = inclusive;
    __syncthreads();
    int64_t before = 0;
    total = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        const int64_t x = lds[w];
        before += w < wave ? x : 0;
        total += x;
    }
    __syncthreads();
    return before + inclusive - value;
}

__global__ __launch_bounds__(kBlock) void k_scan_reduce(const int32_t* in, int64_t n, int64_t* sums) {
    __shared__ int64_t lds[kBlock];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
    int64_t local = 0;
    for (int i = 0; i < kScanItems; ++i) {
        const int64_t idx = base + static_cast<int64_t>(threadIdx.x) * kScanItems + i;
        if (idx < n) local += in[idx];
    }
    int64_t total;
    (void)block_exclusive_scan(local, lds, total);
    if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

__global__ __launch_bounds__(kBlock) void k_scan_blocks(int64_t* sums, int64_t nb) {
    __shared__ int64_t lds[kBlock];
    int64_t carry = 0;
    for (int64_t base = 0; base < nb; base += kBlock) {
        const int64_t idx = base + threadIdx.x;
        const int64_t v = idx < nb ? sums[idx] : 0;
        int64_t total;
        const int64_t ex = block_exclusive_scan(v, lds, total);
        if (idx < nb) sums[idx] = carry + ex;
        carry += total;
    }
    if (threadIdx.x == 0) sums[nb] = carry;
}

__global__ __launch_bounds__(kBlock) void k_scan_apply(const int32_t* in, int64_t n, const int64_t* sums,
                                                       int64_t nb, int64_t* out) {
    __shared__ int64_t lds[kBlock];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
    int64_t vals[kScanItems];
    int64_t local = 0;
    for (int i = 0; i < kScanItems; ++i) {
        const int64_t idx = base + static_cast<int64_t>(threadIdx.x) * kScanItems + i;
        vals[i] = idx < n ? in[idx] : 0;
        local += vals[i];
    }
    int64_t total;
    int64_t run = sums[blockIdx.x] + block_exclusive_scan(local, lds, total);
    for (int i = 0; i < kScanItems; ++i) {
        const int64_t idx = base + static_cast<int64_t>(threadIdx.x) * kScanItems + i;
        if (idx < n) out[idx] = run;
        run += vals[i];
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) out[n] = sums[nb];
}

// the whole scan in one workgroup of 1,024 threads, tile after tile (short
// arrays, up to 8,192 entries a tile: one launch instead of three, and for
// the graph's cell counts one tile instead of three of 2,048)
constexpr int kScanOneThreads = 1024;
constexpr int kScanOneTile = kScanOneThreads * kScanItems;
__global__ __launch_bounds__(kScanOneThreads) void k_scan_one(const int32_t* in, int64_t n, int64_t* out) {
    __shared__ int64_t lds[kScanOneThreads / kWave];
    int64_t carry = 0;
    for (int64_t base = 0; base < n; base += kScanOneTile) {
        int64_t vals[kScanItems];
        int64_t local = 0;
        for (int i = 0; i < kScanItems; ++i) {
            const int64_t idx = base + static_cast<int64_t>(threadIdx.x) * kScanItems + i;
            vals[i] = idx < n ? in[idx] : 0;
            local += vals[i];
        }
        int64_t total;
        int64_t run = carry + block_exclusive_scan<kScanOneThreads>(local, lds, total);
        for (int i = 0; i < kScanItems; ++i) {
            const int64_t idx = base + static_cast<int64_t>(threadIdx.x) * kScanItems + i;
            if (idx < n) out[idx] = run;
            run += vals[i];
        }
        carry += total;
    }
    if (threadIdx.x == 0) out[n] = carry;
}

constexpr int64_t kScanOneTiles = 8; // up to 8 tiles of kScanTile (2 of kScanOneTile): one workgroup

unsigned grid_for(int64_t work, int block = kBlock) {
    const int64_t blocks = (work + block - 1) / block;
    return static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(blocks, 1 << 20)));
}

} // namespace

void scan_counts(hipStream_t stream, const int32_t* in, int64_t* out, int64_t n, DeviceBuffer& tmp) {
    const int64_t nb = std::max<int64_t>(1, (n + kScanTile - 1) / kScanTile);
    if (nb <= kScanOneTiles) {
        hipLaunchKernelGGL(k_scan_one, dim3(1), dim3(kScanOneThreads), 0, stream, in, n, out);
        return;
    }
    tmp.reserve(static_cast<size_t>(nb + 1) * sizeof(int64_t));
    int64_t* sums = tmp.as<int64_t>();
    hipLaunchKernelGGL(k_scan_reduce, dim3(static_cast<unsigned>(nb)), dim3(kBlock), 0, stream, in, n, sums);
    hipLaunchKernelGGL(k_scan_blocks, dim3(1), dim3(kBlock), 0, stream, sums, nb);
    hipLaunchKernelGGL(k_scan_apply, dim3(static_cast<unsigned>(nb)), dim3(kBlock), 0, stream, in, n, sums, nb,
                       out);
    MDX_HIP(hipGetLastError());
}

void prepare_batch(const mdx_batch_view& batch, const int32_t* species, int n_species, double cutoff,
                   PreparedBatch& out) {
    if (!std::isfinite(cutoff) || cutoff <= 0.0) {
        throw Error(MDX_INVALID_ARGUMENT, "neighbor cutoff must be finite and positive");
    }
    validate_batch(batch);
    if (batch.atoms > std::numeric_limits<int32_t>::max()) {
        throw Error(MDX_INVALID_ARGUMENT, "neighbor atom index exceeds int32 range");
    }
    out.structures = batch.structures;
    out.atoms = batch.atoms;
    out.cutoff = cutoff;
    out.n_species = species != nullptr ? n_species : 1;
    out.offsets.assign(batch.offsets, batch.offsets + batch.structures + 1);
    out.types.assign(static_cast<size_t>(batch.atoms), 0);
    if (species != nullptr) {
        std::unordered_map<int32_t, int32_t> map;
        for (int t = 0; t < n_species; ++t) map.emplace(species[t], t);
        for (int64_t i = 0; i < batch.atoms; ++i) {
            const auto it = map.find(batch.numbers[i]);
            if (it == map.end()) {
                throw Error(MDX_INVALID_ARGUMENT, "batch contains an atomic number outside calculator species");
            }
            out.types[static_cast<size_t>(i)] = it->second;
        }
    }
    out.geom.assign(static_cast<size_t>(batch.structures), StructGeom{});
    out.atom_struct.resize(static_cast<size_t>(batch.atoms));
    for (int64_t s = 0; s < batch.structures; ++s) {
        std::fill(out.atom_struct.begin() + batch.offsets[s], out.atom_struct.begin() + batch.offsets[s + 1],
                  static_cast<int32_t>(s));
    }
    out.images.clear();
    out.most_images = 0;
    out.max_images = 1;
    out.chunk_bound = 0;
    int64_t ext = 0;
    for (int64_t s = 0; s < batch.structures; ++s) {
        StructGeom& g = out.geom[static_cast<size_t>(s)];
        std::memset(&g, 0, sizeof(g));
        const int64_t begin = batch.offsets[s];
        const int64_t natoms = batch.offsets[s + 1] - begin;
        g.atom_begin = begin;
        g.natoms = static_cast<int32_t>(natoms);
        g.ext_begin = ext;
        g.image_begin = static_cast<int64_t>(out.images.size());
        const double* cell = batch.cells + s * 9;
        const bool periodic = batch.pbc[s * 3] == 1;
        int bounds[3] = {0, 0, 0};
        if (periodic) {
            double inv[9];
            if (!inverse3(cell, inv)) throw Error(MDX_INVALID_ARGUMENT, "cell matrix is singular");
            for (int a = 0; a < 3; ++a) {
                // neighbor.cpp:459-467
                const double bound = std::floor(
                    cutoff * std::sqrt(inv[0 * 3 + a] * inv[0 * 3 + a] + inv[1 * 3 + a] * inv[1 * 3 + a]
                                       + inv[2 * 3 + a] * inv[2 * 3 + a])
                    + 1.0);
                if (!std::isfinite(bound) || bound < 0.0 || bound > 1024.0) {
                    throw Error(MDX_INVALID_ARGUMENT, "periodic image range exceeds the device graph capacity");
                }
                bounds[a] = static_cast<int>(bound);
            }
        }
        const int64_t n_images = static_cast<int64_t>(2 * bounds[0] + 1) * (2 * bounds[1] + 1) * (2 * bounds[2] + 1);
        if (natoms * n_images > std::numeric_limits<int32_t>::max()) {
            throw Error(MDX_INVALID_ARGUMENT, "periodic images exceed the device graph capacity");
        }
        g.n_images = static_cast<int32_t>(n_images);
        for (int n0 = -bounds[0]; n0 <= bounds[0]; ++n0) {
            for (int n1 = -bounds[1]; n1 <= bounds[1]; ++n1) {
                for (int n2 = -bounds[2]; n2 <= bounds[2]; ++n2) {
                    ImageDesc im{};
                    for (int a = 0; a < 3; ++a) {
                        // Vec3 shift = n0*row0 + n1*row1 + n2*row2 (neighbor.cpp:472-474)
                        im.shift[a] = periodic ? (static_cast<double>(n0) * cell[0 * 3 + a]
                                                  + static_cast<double>(n1) * cell[1 * 3 + a])
                                                     + static_cast<double>(n2) * cell[2 * 3 + a]
                                               : 0.0;
                    }
                    im.n[0] = n0;
                    im.n[1] = n1;
                    im.n[2] = n2;
                    out.images.push_back(im);
                }
            }
        }
        // the extreme shifts per axis: the frame's bounding box of every image
        // (build_grid, neighbor.cpp:143-158) is the atoms' box moved by them
        for (int a = 0; a < 3; ++a) {
            double lo = 0.0, hi = 0.0;
            for (int64_t q = 0; q < n_images; ++q) {
                const double sh = out.images[static_cast<size_t>(g.image_begin + q)].shift[a];
                if (q == 0 || sh < lo) lo = sh;
                if (q == 0 || sh > hi) hi = sh;
            }
            g.shift_lo[a] = lo;
            g.shift_hi[a] = hi;
        }
        out.max_images = std::max(out.max_images, static_cast<int>(n_images));
        if (natoms == 0) continue;
        const int64_t images = natoms * n_images;
        ext += images;
        out.most_images = std::max(out.most_images, images);
        out.chunk_bound += (images + kBinChunk - 1) / kBinChunk;
    }
    if (ext >= (int64_t(1) << 32) - 1) {
        throw Error(MDX_INVALID_ARGUMENT, "periodic images exceed the device graph capacity");
    }
    out.ext_total = ext;
    frame_items(out);
    out.cells_total = out.wave_cells = out.big_bound = out.chunks = out.small_structs = out.large_structs = 0;
    out.direct_bins = out.struct_bins = false;
}

void upload_batch(hipStream_t stream, const mdx_batch_view& batch, PreparedBatch& pb) {
    const size_t atoms = static_cast<size_t>(pb.atoms);
    pb.d_positions.reserve(std::max<size_t>(1, atoms * 3 * sizeof(double)));
    pb.d_types.reserve(std::max<size_t>(1, atoms * sizeof(int32_t)));
    pb.d_atom_struct.reserve(std::max<size_t>(1, atoms * sizeof(int32_t)));
    pb.d_geom.reserve(std::max<size_t>(1, pb.geom.size() * sizeof(StructGeom)));
    pb.d_images.reserve(std::max<size_t>(1, pb.images.size() * sizeof(ImageDesc)));
    pb.d_offsets.reserve(pb.offsets.size() * sizeof(int64_t));
    size_frame(pb);
    if (!pb.frame_items.empty()) {
        MDX_HIP(hipMemcpyAsync(pb.d_frame_items.ptr, pb.frame_items.data(), pb.frame_items.size() * sizeof(FrameItem),
                               hipMemcpyHostToDevice, stream));
    }
    MDX_HIP(hipMemcpyAsync(pb.d_frame_item_start.ptr, pb.frame_item_start.data(),
                           pb.frame_item_start.size() * sizeof(int64_t), hipMemcpyHostToDevice, stream));
    if (!pb.frame_fused.empty()) {
        MDX_HIP(hipMemcpyAsync(pb.d_frame_lists.ptr, pb.frame_fused.data(), pb.frame_fused.size() * sizeof(int32_t),
                               hipMemcpyHostToDevice, stream));
    }
    if (!pb.frame_large.empty()) {
        MDX_HIP(hipMemcpyAsync(pb.d_frame_lists.as<int32_t>() + pb.frame_fused.size(), pb.frame_large.data(),
                               pb.frame_large.size() * sizeof(int32_t), hipMemcpyHostToDevice, stream));
    }
    if (atoms > 0) {
        MDX_HIP(hipMemcpyAsync(pb.d_positions.ptr, batch.positions, atoms * 3 * sizeof(double),
                               hipMemcpyHostToDevice, stream));
        MDX_HIP(hipMemcpyAsync(pb.d_types.ptr, pb.types.data(), atoms * sizeof(int32_t), hipMemcpyHostToDevice,
                               stream));
        MDX_HIP(hipMemcpyAsync(pb.d_atom_struct.ptr, pb.atom_struct.data(), atoms * sizeof(int32_t),
                               hipMemcpyHostToDevice, stream));
    }
    if (!pb.geom.empty()) {
        MDX_HIP(hipMemcpyAsync(pb.d_geom.ptr, pb.geom.data(), pb.geom.size() * sizeof(StructGeom),
                               hipMemcpyHostToDevice, stream));
    }
    if (!pb.images.empty()) {
        MDX_HIP(hipMemcpyAsync(pb.d_images.ptr, pb.images.data(), pb.images.size() * sizeof(ImageDesc),
                               hipMemcpyHostToDevice, stream));
    }
    MDX_HIP(hipMemcpyAsync(pb.d_offsets.ptr, pb.offsets.data(), pb.offsets.size() * sizeof(int64_t),
                           hipMemcpyHostToDevice, stream));
    // pageable sources: the copies are staged synchronously by the runtime,
    // but wait so the host vectors may change after return
    MDX_HIP(hipStreamSynchronize(stream));
}

namespace {

// rows and largest row count over the statistics lines; every centre must
// have been searched (the host's list of home cells holding centres and the
// device's placement of the centres agree)
// binned images: the multi-kernel binning's total, or the per-structure
// binnings' counts spread over the statistics lines
int64_t binned_total(const unsigned long long* st) {
    int64_t binned = static_cast<int64_t>(st[kStatBinned]);
    for (int l = 0; l < kStatLanes; ++l) binned += static_cast<int64_t>(st[stat_binned(l)]);
    return binned;
}

void reduce_stats(const unsigned long long* st, int64_t atoms, int64_t& rows, int64_t& most) {
    rows = 0;
    most = 0;
    int64_t centres = 0;
    for (int l = 0; l < kStatLanes; ++l) {
        rows += static_cast<int64_t>(st[stat_rows(l)]);
        most = std::max(most, static_cast<int64_t>(st[stat_most(l)]));
        centres += static_cast<int64_t>(st[stat_centres(l)]);
    }
    if (centres != atoms) throw Error(MDX_INTERNAL, "the neighbour search missed a centre's home cell");
}

} // namespace

int64_t build_graph(hipStream_t stream, PreparedBatch& pb, DeviceGraph& gr, const volatile int32_t* cancel,
                    bool slotted, bool defer_stats, bool reuse_frame) {
    gr.stats_pending = false;
    const int S = pb.n_species;
    gr.n_species = S;
    const int64_t atoms = pb.atoms;
    gr.pair_start.reserve(static_cast<size_t>(atoms + 1) * sizeof(int64_t));
    gr.slots = 0;
    // the position-dependent inputs: grid, regions of interest, binning
    // paths, centres by home cell and search lists, on the device (one host
    // round trip); it leaves the counter block cleared
    if (!reuse_frame) prepare_frame(stream, pb, gr);
    const int64_t cells = pb.cells_total;
    if (atoms == 0 || cells == 0) {
        MDX_HIP(hipMemsetAsync(gr.pair_start.ptr, 0, static_cast<size_t>(atoms + 1) * sizeof(int64_t), stream));
        gr.counts.reserve(std::max<size_t>(1, static_cast<size_t>(atoms * S) * sizeof(int32_t)));
        gr.pairs = 0;
        gr.binned = 0;
        gr.most_rows = gr.row_bound = 0;
        return 0;
    }
    const size_t cells1 = static_cast<size_t>(cells + 1);
    const StructGeom* geom = pb.d_geom.as<StructGeom>();
    const ImageDesc* images = pb.d_images.as<ImageDesc>();
    const double* pos = pb.d_positions.as<double>();
    const int64_t ext = pb.ext_total;
    if (ext >= (int64_t(1) << 31)) {
        // a centre's candidates are counted in 32-bit integers
        throw Error(MDX_INVALID_ARGUMENT, "periodic images exceed the device graph capacity");
    }

    // the zero-filled counter block: search statistics, then the cell
    // counters of binning (count, fill) and the centres of each home cell
    const int64_t capacity = gr.cell_capacity;
    if (reuse_frame) MDX_HIP(hipMemsetAsync(gr.counters.ptr, 0, graph_counter_bytes(capacity), stream));
    unsigned long long* stats = gr.counters.as<unsigned long long>();
    int32_t* cell_count = graph_cell_counters(gr, capacity, 0);
    int32_t* cell_fill = graph_cell_counters(gr, capacity, 1);
    gr.cell_start.reserve(cells1 * sizeof(int64_t));
    gr.cell_runs.reserve(std::max<size_t>(1, static_cast<size_t>(cells) * static_cast<size_t>(S + 1)) *
                         sizeof(int64_t));
    gr.bin_key.reserve(static_cast<size_t>(ext) * sizeof(uint64_t));
    gr.bin_x.reserve(static_cast<size_t>(ext) * sizeof(double));
    gr.bin_y.reserve(static_cast<size_t>(ext) * sizeof(double));
    gr.bin_z.reserve(static_cast<size_t>(ext) * sizeof(double));
    gr.bin_atom.reserve(static_cast<size_t>(ext) * sizeof(int32_t));
    gr.bin_image.reserve(static_cast<size_t>(ext) * sizeof(int32_t));
    gr.bin_type.reserve(static_cast<size_t>(ext) * sizeof(int32_t));
    gr.counts.reserve(static_cast<size_t>(atoms * S) * sizeof(int32_t));
    gr.totals.reserve(static_cast<size_t>(atoms) * sizeof(int32_t));

    // bin every periodic image into its ROI cell, sorted by (species, extended index)
    if (pb.struct_bins) {
        // each structure on its own: no scan, sort or run search between kernels
        const int32_t* list = pb.d_struct_list.as<int32_t>();
        const int64_t small = pb.small_structs;
        const int64_t large = pb.large_structs;
        if (small > 0) {
            constexpr int64_t per_block = kBlock / kWave;
            hipLaunchKernelGGL(k_bin_small, dim3(static_cast<unsigned>((small + per_block - 1) / per_block)),
                               dim3(kBlock), 0, stream, list, small, geom, images, pos, pb.d_types.as<int32_t>(), S,
                               gr.bin_x.as<double>(), gr.bin_y.as<double>(), gr.bin_z.as<double>(),
                               gr.bin_atom.as<int32_t>(), gr.bin_image.as<int32_t>(), gr.bin_type.as<int32_t>(),
                               gr.cell_runs.as<int64_t>(), stats);
        }
        if (large > 0) {
            hipLaunchKernelGGL(k_bin_struct, dim3(static_cast<unsigned>(large)), dim3(kStructThreads), 0, stream,
                               list + small, geom, images, pos, pb.d_types.as<int32_t>(), S, gr.bin_x.as<double>(),
                               gr.bin_y.as<double>(), gr.bin_z.as<double>(), gr.bin_atom.as<int32_t>(),
                               gr.bin_image.as<int32_t>(), gr.bin_type.as<int32_t>(), gr.cell_runs.as<int64_t>(),
                               stats);
        }
    } else {
        const int max_images = pb.max_images;
        const dim3 bin_grid(static_cast<unsigned>(std::min<int64_t>((atoms + kBlock - 1) / kBlock, 1 << 16)),
                            static_cast<unsigned>(std::min(max_images, 65535)));
        const unsigned chunk_grid = static_cast<unsigned>(pb.chunks);
        const int64_t* chunks = pb.d_struct_chunks.as<int64_t>();
        const int species_major = S > 1 ? 1 : 0;
        if (pb.direct_bins) {
            hipLaunchKernelGGL(k_bin_atoms<false>, bin_grid, dim3(kBlock), 0, stream, geom, images, pos,
                               pb.d_atom_struct.as<int32_t>(), pb.d_types.as<int32_t>(), 0, atoms, max_images, cell_count,
                               static_cast<const int64_t*>(nullptr), static_cast<uint64_t*>(nullptr));
        }
        if (chunk_grid > 0) {
            hipLaunchKernelGGL(k_bin_lds<false>, dim3(chunk_grid), dim3(kBinThreads), 0, stream, chunks,
                               pb.structures, geom, images, pos,
                               pb.d_types.as<int32_t>(), 0, cell_count, static_cast<const int64_t*>(nullptr),
                               static_cast<uint64_t*>(nullptr));
        }
        scan_counts(stream, cell_count, gr.cell_start.as<int64_t>(), cells, gr.scan_tmp);
        if (pb.direct_bins) {
            hipLaunchKernelGGL(k_bin_atoms<true>, bin_grid, dim3(kBlock), 0, stream, geom, images, pos,
                               pb.d_atom_struct.as<int32_t>(), pb.d_types.as<int32_t>(), species_major, atoms, max_images,
                               cell_fill, gr.cell_start.as<int64_t>(), gr.bin_key.as<uint64_t>());
        }
        if (chunk_grid > 0) {
            hipLaunchKernelGGL(k_bin_lds<true>, dim3(chunk_grid), dim3(kBinThreads), 0, stream, chunks,
                               pb.structures, geom, images, pos,
                               pb.d_types.as<int32_t>(), species_major, cell_fill, gr.cell_start.as<int64_t>(),
                               gr.bin_key.as<uint64_t>());
        }
        const unsigned cell_grid = static_cast<unsigned>(std::min<int64_t>(cells, 1 << 20));
        // a wavefront per cell when cells hold a wavefront of images on average
        const int sort_threads = ext <= static_cast<int64_t>(kWave) * cells ? kWave : kBlock;
        hipLaunchKernelGGL(k_bin_sort, dim3(cell_grid), dim3(sort_threads), 0, stream, geom,
                           gr.cell_struct.as<int32_t>(), images, pos, pb.d_types.as<int32_t>(), gr.cell_start.as<int64_t>(),
                           cells, gr.bin_key.as<uint64_t>(), gr.bin_x.as<double>(), gr.bin_y.as<double>(),
                           gr.bin_z.as<double>(), gr.bin_atom.as<int32_t>(), gr.bin_image.as<int32_t>(),
                           gr.bin_type.as<int32_t>(), stats);
        hipLaunchKernelGGL(k_cell_species, dim3(grid_for(cells * (S + 1))), dim3(kBlock), 0, stream,
                           gr.cell_start.as<int64_t>(), cells, gr.bin_type.as<int32_t>(), S, gr.cell_runs.as<int64_t>());
    }
    MDX_HIP(hipGetLastError());
    if (cancel != nullptr && *cancel != 0) throw Error(MDX_CANCELLED, "descriptor computation was cancelled");

    // d^2 < c^2 is d^2 <= the largest double below c^2
    const double cutoff2 = pb.cutoff * pb.cutoff;
    const double accept_max = pb.include_boundary ? cutoff2 : std::nextafter(cutoff2, 0.0);
    // cells searched by whole workgroups: the list after the wavefront
    // cells, whose length the frame counted on the device (at most
    // big_bound: workgroups past it return at once)
    const int64_t wave_cells = pb.wave_cells;
    const int32_t* lists = pb.d_cell_lists.as<int32_t>();
    const int64_t big_bound = pb.big_bound;
    const int32_t* big_list = lists + wave_cells;
    const unsigned long long* big_count = reinterpret_cast<const unsigned long long*>(
        static_cast<const char*>(pb.d_frame.ptr) + pb.frame_summary) + kFrameBigCells;
    auto neighbors = [&](auto mode, int64_t cap) {
        if (big_bound > 0) {
            const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(big_bound, 1 << 20));
            hipLaunchKernelGGL(k_neighbors<decltype(mode)::value>, dim3(blocks), dim3(kNbrThreads), 0, stream, geom,
                               gr.cell_struct.as<int32_t>(), pos, big_list, big_count,
                               gr.cell_centre_start.as<int64_t>(), pb.d_cell_centres.as<int32_t>(),
                               gr.cell_runs.as<int64_t>(),
                               gr.bin_x.as<double>(), gr.bin_y.as<double>(), gr.bin_z.as<double>(), S, accept_max,
                               gr.counts.as<int32_t>(), gr.totals.as<int32_t>(), gr.pair_start.as<int64_t>(),
                               gr.pair_bin.as<uint32_t>(), cap, stats);
        }
        if (wave_cells > 0) {
            constexpr int64_t per_block = kBlock / kWave;
            const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((wave_cells + per_block - 1) / per_block,
                                                                            1 << 20));
            hipLaunchKernelGGL(k_neighbors_wave<decltype(mode)::value>, dim3(blocks), dim3(kBlock), 0, stream, lists,
                               wave_cells, pos, gr.cell_centre_start.as<int64_t>(), pb.d_cell_centres.as<int32_t>(),
                               gr.cell_runs.as<int64_t>(),
                               gr.bin_x.as<double>(), gr.bin_y.as<double>(), gr.bin_z.as<double>(), S, accept_max,
                               gr.counts.as<int32_t>(), gr.totals.as<int32_t>(), gr.pair_start.as<int64_t>(),
                               gr.pair_bin.as<uint32_t>(), cap, stats);
        }
        MDX_HIP(hipGetLastError());
    };
    using Count = std::integral_constant<int, kNbrCount>;
    using Fill = std::integral_constant<int, kNbrFill>;
    using Slotted = std::integral_constant<int, kNbrSlotted>;
    // slots no wider than the most rows a centre can have (a structure's
    // binned images), in whole 64-byte lines: small structures keep their
    // rows close together
    const int64_t cap = slotted ? std::min(gr.slot_cap, std::max<int64_t>(16, (pb.most_images + 15) / 16 * 16)) : 0;
    const int64_t slot_bytes = atoms * cap * static_cast<int64_t>(sizeof(uint32_t));
    // from an arena, the slotted layout only when its rows fit in what is left
    ScratchArena* arena = gr.pair_bin.arena;
    const bool use_slots = cap > 0 && slot_bytes <= kMaxSlottedBytes &&
                           (arena == nullptr || static_cast<size_t>(slot_bytes) <= arena->left());
    gr.slots = 0;
    if (use_slots) {
        // one pass: counts and rows at centre * cap; a reservation four times
        // what is needed and over 256 MiB (left by a denser batch) goes back
        const size_t need = static_cast<size_t>(atoms * cap) * sizeof(uint32_t);
        if (arena == nullptr && gr.pair_bin.bytes > 4 * need && gr.pair_bin.bytes > (size_t(256) << 20)) {
            gr.pair_bin.release();
        }
        gr.pair_bin.reserve(need);
        neighbors(Slotted{}, cap);
        unsigned long long* st = gr.stats_host.get(kStatWords);
        MDX_HIP(hipMemcpyAsync(st, stats, kStatWords * sizeof(unsigned long long), hipMemcpyDeviceToHost, stream));
        if (defer_stats && arena == nullptr) {
            // the consumer is launched before the statistics are read
            // (complete_graph); until then every centre counts as fitting.
            // Not from an arena: a rebuild after an overflow would need the
            // space of the pieces taken after the slotted rows.
            gr.read_back.record(stream);
            gr.stats_pending = true;
            gr.slots = cap;
            gr.most_rows = 0;
            gr.row_bound = cap;
            gr.pairs = -1;
            gr.binned = -1;
            return -1;
        }
        // the expansion launch waits on these words: poll rather than sleep in
        // a blocking synchronisation, whose wake-up costs tens of microseconds
        gr.read_back.wait(stream);
        if (cancel != nullptr && *cancel != 0) throw Error(MDX_CANCELLED, "descriptor computation was cancelled");
        int64_t pairs = 0, most = 0;
        reduce_stats(st, atoms, pairs, most);
        const int64_t binned = binned_total(st);
        gr.most_rows = most;
        gr.row_bound = most;
        if (most <= cap) {
            // slots grown for a denser batch shrink back to what fits this one
            int64_t fit = kMinSlotCap;
            while (fit < most) fit *= 2;
            if (fit < gr.slot_cap) gr.slot_cap = fit;
            gr.slots = cap;
            gr.pairs = pairs;
            gr.binned = binned;
            return pairs;
        }
        // a centre overflowed its slot: later calls use a larger one (or the
        // compact layout), this one lays the counted rows out compactly
        int64_t grown = kMinSlotCap;
        while (grown < most) grown *= 2;
        gr.slot_cap = grown <= kMaxSlotCap ? grown : 0;
        if (arena != nullptr) {
            // the slotted rows were the arena's last piece and are not read
            // again: the compact rows reuse their space
            arena->rewind(gr.pair_bin.ptr);
            gr.pair_bin.ptr = nullptr;
            gr.pair_bin.bytes = 0;
        }
        // the slotted pass cut the overflowing centres' per-species counts to
        // their slots: a count pass writes the true ones (the fill pass writes
        // rows only)
        neighbors(Count{}, 0);
        scan_counts(stream, gr.totals.as<int32_t>(), gr.pair_start.as<int64_t>(), atoms, gr.scan_tmp);
        gr.pair_bin.reserve(std::max<size_t>(1, static_cast<size_t>(pairs) * sizeof(uint32_t)));
        neighbors(Fill{}, 0);
        gr.pairs = pairs;
        gr.binned = binned;
        return pairs;
    }
    neighbors(Count{}, 0);
    scan_counts(stream, gr.totals.as<int32_t>(), gr.pair_start.as<int64_t>(), atoms, gr.scan_tmp);
    MDX_HIP(hipGetLastError());
    int64_t pairs = 0;
    MDX_HIP(hipMemcpyAsync(&pairs, gr.pair_start.as<int64_t>() + atoms, sizeof(int64_t), hipMemcpyDeviceToHost,
                           stream));
    unsigned long long st[kStatWords] = {};
    MDX_HIP(hipMemcpyAsync(st, stats, sizeof(st), hipMemcpyDeviceToHost, stream));
    MDX_HIP(hipStreamSynchronize(stream));
    const int64_t binned = binned_total(st);
    int64_t counted = 0;
    reduce_stats(st, atoms, counted, gr.most_rows);
    gr.row_bound = gr.most_rows;
    if (slotted && gr.slot_cap == 0 && gr.most_rows <= kMaxSlotCap) {
        // the slotted layout again once a batch's centres fit a slot
        int64_t fit = kMinSlotCap;
        while (fit < gr.most_rows) fit *= 2;
        gr.slot_cap = fit;
    }
    if (cancel != nullptr && *cancel != 0) throw Error(MDX_CANCELLED, "descriptor computation was cancelled");
    if (pairs >= (int64_t(1) << 40)) throw Error(MDX_INTERNAL, "implausible neighbour pair count");
    gr.pair_bin.reserve(std::max<size_t>(1, static_cast<size_t>(pairs) * sizeof(uint32_t)));
    neighbors(Fill{}, 0);
    gr.pairs = pairs;
    gr.binned = binned;
    return pairs;
}

bool complete_graph(const PreparedBatch& pb, DeviceGraph& gr, const volatile int32_t* cancel) {
    if (!gr.stats_pending) return true;
    gr.stats_pending = false;
    gr.read_back.sync();
    const unsigned long long* st = gr.stats_host.get(kStatWords);
    int64_t pairs = 0, most = 0;
    reduce_stats(st, pb.atoms, pairs, most);
    if (cancel != nullptr && *cancel != 0) throw Error(MDX_CANCELLED, "descriptor computation was cancelled");
    gr.binned = binned_total(st);
    gr.most_rows = most;
    gr.row_bound = most;
    gr.pairs = pairs;
    const int64_t cap = gr.slots;
    if (most <= cap) {
        // slots grown for a denser batch shrink back to what fits this one
        int64_t fit = kMinSlotCap;
        while (fit < most) fit *= 2;
        if (fit < gr.slot_cap) gr.slot_cap = fit;
        return true;
    }
    // a centre overflowed its slot: later builds use a larger one (or the
    // compact layout); this batch is built again by the caller
    int64_t grown = kMinSlotCap;
    while (grown < most) grown *= 2;
    gr.slot_cap = grown <= kMaxSlotCap ? grown : 0;
    gr.slots = 0;
    return false;
}

} // namespace mdx
