// Internal declarations shared by the gfx950 translation units of the SOAP
// library.  Compiled with -ffp-contract=off: every fused multiply-add in the
// device code is written out with fma(), so the geometry arithmetic
// (image shifts, displacements, squared distances) rounds exactly like the
// reference's C++ (cpp/src/common/neighbor.cpp:471-478, 569;
// cpp/include/mdescriptor/detail/math3.hpp:19-35).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <functional>
#include <mutex>
#include <stdexcept>
#include <string>
#include <memory>
#include <vector>

#include "../../include/mdx_hip.h"

namespace mdx {

constexpr int kMaxSpecies = 16;   // species per SOAP plan handled on the device
constexpr int kMaxNmax = 16;      // radial channels per (species, l)
constexpr int kMaxLmax = 20;      // as the reference's parameter check (soap.cpp:1153-1154)
constexpr int kBlock = 256;       // threads per workgroup of the graph and SOAP kernels
constexpr int kWave = 64;         // CDNA wavefront width

// Error carrying one of the C-ABI status codes; thrown inside the library and
// converted to a status at the extern "C" boundary.
struct Error : std::runtime_error {
    int status;
    Error(int code, const std::string& message) : std::runtime_error(message), status(code) {}
};

void check_hip(hipError_t code, const char* what);
#define MDX_HIP(call) ::mdx::check_hip((call), #call)

// Bump allocator over a caller-owned block of device memory (the library's
// static scratch array).  take() hands out 256-byte aligned pieces and throws
// MDX_INVALID_ARGUMENT when the block is exhausted; rewind(p) gives back p
// and every piece taken after it; reset() starts over.
struct ScratchArena {
    char* base = nullptr;
    size_t capacity = 0;
    size_t used = 0;
    void* take(size_t size);
    void rewind(void* piece);
    size_t left() const { return capacity - used; }
    void reset() { used = 0; }
};

// Grow-only device buffer.  Reallocated only when a larger size is asked for.
// A buffer bound to an arena takes its memory from it instead and never
// allocates or frees device memory.
struct DeviceBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
    ScratchArena* arena = nullptr;
    void reserve(size_t size);
    void release();
    template <typename T> T* as() const { return static_cast<T*>(ptr); }
    ~DeviceBuffer() { release(); }
    DeviceBuffer() = default;
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
};

// One structure's cell-grid geometry, as seen by the device.  The grid is the
// reference's (build_grid, neighbor.cpp:135-194) over every periodic image of
// the structure; only the box of cells within one cell of a centre (the
// "region of interest") is materialised.
struct StructGeom {
    int64_t atom_begin;  // first atom of the structure in the batch
    int64_t ext_begin;   // first index of the structure in image-major enumeration space
    int64_t cell_begin;  // first global ROI cell of the structure
    int64_t image_begin; // first entry of the structure in the image table
    int32_t natoms;
    int32_t n_images;
    int32_t dims[3];     // full grid dimensions
    int32_t roi_lo[3];   // ROI box origin (grid coordinates)
    int32_t roi_dim[3];  // ROI box extent
    int32_t one_cell;    // 1: the ROI is one cell holding every image, at most a wavefront of them
    int32_t lds_bins;    // 1: binned by workgroups counting in LDS over the ROI cells (kLdsBinCells or fewer)
    int32_t reserved;
    double minimum[3];   // grid origin (bounding box minus padding)
    double spacing[3];   // cell widths
    // smallest and largest image shift per axis (topology: fixed with the
    // cell); the bounding box of every image is the atoms' box moved by them
    double shift_lo[3];
    double shift_hi[3];
};

// Binning paths and their limits (kernel 1).  Which path a structure takes
// depends on its region of interest, so on the positions: the frame kernels
// classify every structure on the device each time a graph is built.
constexpr int kLdsBinCells = 2048;     // ROI cells of a structure binned in LDS, at most
constexpr int kBinChunk = 4096;        // images per LDS binning workgroup
constexpr int kStructImages = 8192;    // images of a structure binned by one workgroup, at most
constexpr int kStructMinImages = 1024; // images per such structure, on average, for that path
constexpr int kSmallImages = kWave;    // images of a structure binned by one wavefront, at most
constexpr int kSmallCells = 64;        // ... and its ROI cells
constexpr int kWaveCellImages = kWave; // binned images of a one-cell structure searched by one wavefront

// CellGrid::coordinate (neighbor.cpp:122-132); shared by host and device.
__host__ __device__ inline int grid_coordinate(double value, double origin, double width, int dim) {
    const double scaled = (value - origin) / width;
    if (!(scaled > 0.0)) return 0;
    if (!__builtin_isfinite(scaled) || scaled >= static_cast<double>(dim)) return dim - 1;
    return static_cast<int>(scaled);
}

// A run of one structure's binned images [first, first + count) in extended
// (image-major) order: the work of one binning workgroup.
struct BinChunk {
    int64_t first;
    int32_t structure;
    int32_t count;
};

// A run of at most kItemAtoms atoms of one structure: the unit of work of the
// frame's per-atom kernels (one wavefront each).  64-atom items measured
// slower (config 2 graph 0.304 -> 0.322 ms, config 5 0.513 -> 0.624 ms): the
// last wavefront of a structure reduces 4x the partial results.
struct FrameItem {
    int64_t first;
    int32_t large;   // index of the structure in PreparedBatch::frame_large
    int32_t count;
};
constexpr int kItemAtoms = 256;
// structures of at most this many atoms take their whole frame in one
// wavefront (frame_small in k_frame_first); larger ones are split into items
constexpr int kFuseAtoms = 1024;

// Periodic image: integer shift and its Cartesian vector, computed on the
// host as ((n0*a + n1*b) + n2*c) per component (neighbor.cpp:472-474).
struct ImageDesc {
    double shift[3];
    int32_t n[3];
    int32_t pad;
};

// Page-locked host words for small device-to-host read-backs (a copy into
// pageable memory goes through a staging buffer synchronously).
class PinnedWords {
public:
    PinnedWords() = default;
    PinnedWords(const PinnedWords&) = delete;
    PinnedWords& operator=(const PinnedWords&) = delete;
    ~PinnedWords();
    unsigned long long* get(size_t count); // at least count words, allocated on first use

private:
    unsigned long long* words_ = nullptr;
    size_t count_ = 0;
};

// An event recorded on a stream and polled until the stream reaches it (a
// lower-latency wait than a blocking stream synchronisation).  Created on
// first use on the current device; one per owner, not copyable.
class StreamPoint {
public:
    StreamPoint() = default;
    StreamPoint(const StreamPoint&) = delete;
    StreamPoint& operator=(const StreamPoint&) = delete;
    ~StreamPoint();
    void prepare(); // create the event on the current device now
    void wait(hipStream_t stream); // record, then sync
    void record(hipStream_t stream);
    void sync(); // until the stream reaches the last recorded point

private:
    hipEvent_t event_ = nullptr;
};

// Words of a frame's summary, read back once per graph build after the frame
// kernels have classified the structures (frame.hip).
enum FrameWord {
    kFrameCells = 0,      // ROI cells of the batch
    kFrameWaveCells,      // one-cell structures (searched one wavefront each)
    kFrameChunks,         // LDS binning chunks
    kFrameSmall,          // structures of at most kSmallImages images and kSmallCells ROI cells
    kFrameLarge,          // other structures with atoms
    kFrameLargeFit,       // ... of which fit one binning workgroup
    kFrameLargeImages,    // images of the large structures
    kFrameDirect,         // structures with atoms binned with global atomics
    kFrameBigBound,       // sum over workgroup-searched structures of min(ROI cells, atoms)
    kFrameStatus,         // error bits (kFrameNonFinite, kFrameGridTooLarge)
    kFrameBigCells,       // home cells of workgroup-searched structures that hold centres (counted after the read-back)
    kFrameWords = 16
};
constexpr unsigned long long kFrameNonFinite = 1;   // a position is not finite
constexpr unsigned long long kFrameGridTooLarge = 2; // a grid dimension is not finite or above 1e6 cells

// A structure batch on the device.  Topology (everything fixed by numbers,
// cells, pbc and offsets) is prepared on the host once per batch; everything
// that depends on positions (the cell grid, each structure's region of
// interest and binning path, the centres' home cells and the lists the
// search walks) is rebuilt on the device by the frame kernels at the start of
// every graph build (prepare_frame), so a batch whose positions change keeps
// its topology and only re-runs those kernels.
struct PreparedBatch {
    int64_t structures = 0;
    int64_t atoms = 0;
    int64_t ext_total = 0;   // sum over structures of natoms * n_images
    double cutoff = 0.0;
    int include_boundary = 1;  // d^2 <= cutoff^2 (1) or d^2 < cutoff^2 (0), neighbor.cpp:553-555
    int n_species = 1;
    // topology, host copies (uploaded by upload_batch)
    std::vector<StructGeom> geom; // position-dependent fields zero until a frame fills them on the device
    std::vector<ImageDesc> images;
    std::vector<int32_t> types; // species index per atom (0 when species are ignored)
    std::vector<int32_t> atom_struct; // structure of each atom
    std::vector<int64_t> offsets;
    // work items of the averaged SOAP modes and the folded rows' structure
    // ranges (host copies outlive the async upload)
    std::vector<int64_t> item_begin, struct_items, fold_items;
    int64_t most_images = 0;  // most binned images of one structure: no centre has more rows
    int max_images = 1;       // most periodic images of one structure
    int64_t chunk_bound = 0;  // LDS binning chunks if every structure took that path (a check of the summary)
    std::vector<int32_t> frame_fused;       // structures of at most kFuseAtoms atoms (frame_items())
    std::vector<int32_t> frame_large;       // the others ...
    std::vector<FrameItem> frame_items;     // ... split into atom runs
    std::vector<int64_t> frame_item_start;  // first item of each large structure, [frame_large.size() + 1]
    // the last frame's summary (prepare_frame)
    int64_t cells_total = 0;  // ROI cells over all structures
    int64_t wave_cells = 0;   // one-cell structures: cell_lists[0, wave_cells)
    int64_t big_bound = 0;    // workgroup-searched home cells, at most: cell_lists[wave_cells, ...)
    int64_t chunks = 0;       // LDS binning chunks (bin_chunks)
    int64_t small_structs = 0, large_structs = 0;
    bool direct_bins = false; // some structure is binned with global atomics (k_bin_atoms)
    // every structure is binned on its own, its bins from its first extended
    // index: by a wavefront of k_bin_small (at most 64 images and 64 ROI
    // cells) or a workgroup of k_bin_struct (at most 2,048 ROI cells and 8,192
    // images; those average 1,024 images or more)
    bool struct_bins = false;
    // device copies of the inputs and topology
    DeviceBuffer d_positions; // f64[atoms*3]
    DeviceBuffer d_types;     // i32[atoms]
    DeviceBuffer d_atom_struct; // i32[atoms]
    DeviceBuffer d_geom;      // StructGeom[structures]
    DeviceBuffer d_images;    // ImageDesc[...]
    DeviceBuffer d_offsets;   // i64[structures+1]
    // frame arrays, written on the device by the frame kernels (sized by the
    // topology at upload, so a run allocates none of them):
    //   frame: per item u64 box words [6] (per axis: the largest order key
    //     of -x, then of x) and u32 span words [6] (per axis: ~ smallest and
    //     largest grid coordinate of a centre), then per structure i64 ROI
    //     cells, i32 class bits, i32 chunks, then the list workgroups' sums,
    //     then the summary words [kFrameWords] (cleared at the start of a
    //     frame)
    DeviceBuffer d_frame;
    size_t frame_bytes = 0, frame_span = 0, frame_vol = 0, frame_cls = 0, frame_nch = 0, frame_blocks = 0,
           frame_done = 0, frame_summary = 0;
    bool frame_done_clear = false; // the item counters (frame_done) were cleared since the arrays were sized
    DeviceBuffer d_frame_items;      // FrameItem[frame_items.size()]
    DeviceBuffer d_frame_item_start; // i64[frame_large.size() + 1]
    DeviceBuffer d_frame_lists;      // i32: frame_fused, then frame_large
    DeviceBuffer d_struct_cells; // i64[structures + 1]: first ROI cell of each structure, then the total
    DeviceBuffer d_struct_chunks; // i64[structures + 1]: first LDS binning chunk of each structure, then the total
    DeviceBuffer d_cell_lists;   // i32[structures + atoms]: one-cell structures' cells, then searched home cells
    DeviceBuffer d_struct_list;  // i32[structures]: the k_bin_small structures, then the k_bin_struct ones
    DeviceBuffer d_cell_centres; // i32[atoms]: centres grouped by home cell
    DeviceBuffer d_atom_cell;    // u64[atoms]: grid coordinates of each centre (x | y << 21 | z << 42)
    DeviceBuffer d_atom_home;    // i32[atoms]: home ROI cell
    DeviceBuffer d_atom_rank;    // i32[atoms]: place among its home cell's centres
    PinnedWords frame_host;      // the summary, read back
    StreamPoint frame_read;
};

// Device graph (kernel 1 output).  Pairs are indices into the cell-sorted
// binned image arrays; rows are grouped by neighbour species when
// n_species > 1 and keep the reference's candidate order inside a species.
struct DeviceGraph {
    int64_t binned = 0;
    int64_t pairs = 0;
    int64_t most_rows = 0;   // largest row count of one centre (valid once the statistics are read)
    int64_t row_bound = 0;   // no centre has more rows in the current layout: the slot width while
                             // the statistics are pending, else most_rows (what consumers may read
                             // before complete_graph)
    bool stats_pending = false; // a deferred slotted build whose statistics are not read yet
    int n_species = 1;
    DeviceBuffer counters;   // zero-filled per build: u64 statistics[kStatWords], then i32 cell
                             // counts of binning (count, fill) and the centres of each home
                             // cell, [cells + 1] each
    DeviceBuffer cell_start; // i64[cells + 1] first bin of each ROI cell
    DeviceBuffer cell_centre_start; // i64[cells + 1]: cell c's centres are the batch's
                                    // cell_centres[cell_centre_start[c], cell_centre_start[c + 1])
    DeviceBuffer cell_struct;       // i32[cells]: structure of each ROI cell
    DeviceBuffer bin_key;                           // unsorted u64 keys, (species << 32) | extended index
    DeviceBuffer cell_runs;  // i64[cells * (n_species + 1)]: first bin of each species in a cell, then its end
    DeviceBuffer bin_x, bin_y, bin_z;               // f64 positions of binned images (sorted)
    DeviceBuffer bin_atom;                          // i32 global atom index
    DeviceBuffer bin_image;                         // i32 global image index
    DeviceBuffer bin_type;                          // i32 species index
    DeviceBuffer counts;     // i32[atoms * n_species]
    DeviceBuffer totals;     // i32[atoms]
    DeviceBuffer pair_start; // i64[atoms + 1]: first row of each centre (compact: the
                             // prefix sum of totals, pair_start[atoms] = pairs; slotted: centre * slots)
    DeviceBuffer pair_bin;   // u32 rows: [pairs] compact, [atoms * slots] slotted
    int64_t cell_capacity = 0; // ROI cells the cell arrays (counters, cell_centre_start, cell_struct) hold
    int64_t slots = 0;       // layout of the last build: 0 compact, else rows reserved per centre
    int64_t slot_cap = 512;  // rows per centre for the next slotted build (0: compact only)
    StreamPoint read_back;   // completion of the statistics read-back
    PinnedWords stats_host;  // its destination
    DeviceBuffer scan_tmp;   // block sums of the scans

    template <typename F> void for_each_buffer(F f) {
        for (DeviceBuffer* b : {&counters, &cell_start, &cell_centre_start, &cell_struct, &bin_key, &cell_runs,
                                &bin_x, &bin_y, &bin_z,
                                &bin_atom, &bin_image, &bin_type, &counts, &totals, &pair_start, &pair_bin,
                                &scan_tmp}) {
            f(*b);
        }
    }
};

// Build (or rebuild) the device graph of a prepared batch at pb.cutoff.
// Returns the pair count.  Polls cancel between launches.  slotted: the rows
// may be laid out at centre * graph.slot_cap (one search pass instead of a
// count and a fill pass) when every centre fits; graph.slots records the
// layout built.  Only consumers that read a centre's rows as pair_start[centre]
// onwards, totals[centre] of them (or the per-species counts), may ask for it:
// the SOAP expansion and the NeighborList kernels.
// graph statistics words, read back once per build: binned images in the
// first 128-byte line, then kStatLanes lines of (rows of the search pass, largest
// row count of a centre, centres searched).  The search kernels spread their
// atomics over those lines: atomics on one address serialise across the
// whole device.
constexpr int kStatBinned = 0;
constexpr int kStatLineWords = 16;
constexpr int kStatLanes = 32;
constexpr int kStatWords = kStatLineWords * (1 + kStatLanes);
// The i32 cell counters in a graph's counter block sized for `capacity`
// cells: 0 binning counts, 1 binning fill cursors, 2 centres per home cell.
inline int32_t* graph_cell_counters(DeviceGraph& g, int64_t capacity, int which) {
    return reinterpret_cast<int32_t*>(g.counters.as<unsigned long long>() + kStatWords) + which * (capacity + 1);
}
inline int32_t* graph_centre_counts(DeviceGraph& g, int64_t capacity) { return graph_cell_counters(g, capacity, 2); }
__host__ __device__ constexpr int stat_rows(int lane) { return kStatLineWords * (1 + lane); }
__host__ __device__ constexpr int stat_most(int lane) { return kStatLineWords * (1 + lane) + 1; }
__host__ __device__ constexpr int stat_centres(int lane) { return kStatLineWords * (1 + lane) + 2; }
__host__ __device__ constexpr int stat_binned(int lane) { return kStatLineWords * (1 + lane) + 3; }
constexpr int64_t kMinSlotCap = 512;
constexpr int64_t kMaxSlotCap = 8192;
constexpr int64_t kMaxSlottedBytes = int64_t(4) << 30;
// The frame runs first (prepare_frame) unless reuse_frame: a rebuild of the
// same positions after a slot overflow.
int64_t build_graph(hipStream_t stream, PreparedBatch& pb, DeviceGraph& graph,
                    const volatile int32_t* cancel, bool slotted = false, bool defer_stats = false,
                    bool reuse_frame = false);
// With defer_stats a slotted build returns (-1) before its statistics are
// read: the caller may queue the graph's consumer at once, then calls
// complete_graph, which reads them.  false: a centre overflowed its slot (the
// slotted search clamped its counts to the slot, so the queued consumer read
// only valid rows, with wrong results for it); build the batch again and
// rerun the consumer.
bool complete_graph(const PreparedBatch& pb, DeviceGraph& graph, const volatile int32_t* cancel);

// Compute units of the current device (queried once per process and device).
int device_compute_units();
// LDS bytes one workgroup may use on the current device (queried once per
// process and device; 160 KiB on gfx950)
size_t device_workgroup_lds();

// Exclusive scan of n int32 counts into n+1 int64 offsets (out[n] = total).
void scan_counts(hipStream_t stream, const int32_t* in, int64_t* out, int64_t n, DeviceBuffer& tmp);

// Prepare a batch's topology on the host (validation, species map, image
// tables, per-structure extents) for cutoff; species may be null (all atoms
// one species).  Nothing here depends on positions beyond their validation.
void prepare_batch(const mdx_batch_view& batch, const int32_t* species, int n_species, double cutoff,
                   PreparedBatch& out);
// Upload the topology and the positions, and size the frame arrays.
void upload_batch(hipStream_t stream, const mdx_batch_view& batch, PreparedBatch& pb);

// The frame (frame.hip): from the positions on the device, each structure's
// cell grid (bounding box of its images, dimensions, spacing), region of
// interest and binning path, written into d_geom; the lists of the binning
// and search kernels; the summary, read back into pb (one host round trip);
// then, into the graph, the centres grouped by home cell and the structure of
// every ROI cell (before the read-back when the graph's cell arrays have
// room for this frame's cells, else after it).
// Throws MDX_INVALID_ARGUMENT for non-finite positions or a grid beyond the
// device graph's capacity, with the messages of prepare_batch's checks.
void prepare_frame(hipStream_t stream, PreparedBatch& pb, DeviceGraph& graph);
// The graph's zero-filled counter block for `capacity` cells: statistics,
// then i32 cell counts of binning (count, fill) and the centres of each
// home cell, [capacity + 1] each; its size, and room for it and the other
// cell arrays of the frame.
size_t graph_counter_bytes(int64_t capacity);
void reserve_cells(DeviceGraph& graph, int64_t capacity);
// The frame kernels' atom runs of a batch (prepare_batch), and the sizes of
// its frame arrays (upload_batch), from its topology.
void frame_items(PreparedBatch& pb);
void size_frame(PreparedBatch& pb);


// NeighborList descriptor over a one-species device graph (neighbor_list.hip).
struct NeighborListState {
    int64_t rows = -1;       // kept pairs of the last count, -1 before any
    int full = 1, self_pairs = 0;
    DeviceBuffer kept;       // i32[atoms]: kept pairs per centre
    DeviceBuffer kept_start; // i64[atoms + 1]: first output row per centre
    DeviceBuffer scan_tmp;
};

// Count the pairs each centre keeps under (full, self_pairs) and scan them;
// records `done` after the scan and returns the total (waits for the stream).
int64_t count_neighbor_list(hipStream_t stream, const PreparedBatch& pb, const DeviceGraph& graph, int full,
                            int self_pairs, NeighborListState& list, hipEvent_t done);

// Write the counted list into device memory: table f64[rows*9], values
// f64[rows*4], samples i64[rows*6], offsets i64[structures+1]; null pointers
// are skipped.  Enqueued on stream, not waited for.
void fill_neighbor_list(hipStream_t stream, const PreparedBatch& pb, const DeviceGraph& graph,
                        const NeighborListState& list, double* table, double* values, int64_t* samples,
                        int64_t* offsets);

} // namespace mdx

// Opaque C-ABI objects.
struct mdx_hip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::mutex mutex;
    std::string last_error;
    mdx::PreparedBatch scratch_batch; // used by mdx_hip_soap_compute / neighbors / neighbor_list
    mdx::DeviceGraph graph;
    int graph_kind = 0;               // what last built `graph`: 0 none, 1 SOAP, 2 neighbors, 3 neighbor list
    mdx::NeighborListState list;
    hipEvent_t list_events[5] = {};   // neighbour list: graph start / graph end / count end, fill start / end
    bool list_filled = false;         // a fetch since the last list wrote records
    mdx::DeviceBuffer out_dev;        // device result of mdx_hip_soap_compute
    mdx::DeviceBuffer partials;       // inner/outer partial sums
    void* pinned = nullptr;           // pinned staging ring (two halves) for pageable result downloads
    size_t pinned_bytes = 0;
    hipEvent_t events[8] = {};
    hipEvent_t stage_events[2] = {};  // completion of the DMA into each staging half
    hipStream_t copy_stream = nullptr; // result downloads overlapped with the expansion launches
    hipStream_t graph_stream = nullptr; // pipelined frames: the next frame's graph beside this one's expansion
    std::vector<hipEvent_t> slice_events; // end of each expansion launch, waited on by copy_stream
    mdx::StreamPoint finished;        // end of a device-batch run (polled)
    // mdx_hip_soap_run_noalloc: the device's static scratch array as an arena,
    // and the graph and partial sums that live in it (bound to the arena at
    // context creation, emptied at the start of every call)
    mdx::ScratchArena arena;
    mdx::DeviceGraph static_graph;
    mdx::DeviceBuffer static_partials;
};

struct mdx_soap_plan {
    int device = 0;
    int S = 0, n = 0, l_max = 0, L = 0, H = 0, LN = 0;
    int average = 0, out_dtype = 8;
    double r_cut = 0.0, sigma = 0.0, cutoff = 0.0;
    int64_t features = 0, coeff_size = 0;
    std::vector<int32_t> species;
    mdx::DeviceBuffer d_pref, d_expo, d_beta, d_ps_pref; // radial prefactors/exponents, scaled beta, PS prefactors
    mdx::DeviceBuffer d_feat_a, d_feat_b;                // feature table: (c row offsets, l)
    mdx::DeviceBuffer d_hnorm;                           // harmonic normalisation N_lm (x sqrt(2) for m > 0)
    // matrix-core path (soap_mfma.hip): tile maps, beta-fold operands, feature index tables
    bool use_mfma = false;
    int tiles = 0;
    int hpad = 0;  // padded harmonic row of the matrix-core layout
    int clamp = 0; // 1 when expo * cutoff^2 can exceed 700
    mdx::DeviceBuffer d_row_channel, d_col_harmonic, d_beta_lane, d_fbase, d_fstride;
    // 4x4-block kernel (soap_quad.hip), default options only: wavefronts (0:
    // not used), radial groups, MFMA instructions per step, lane constants
    int quad_waves = 0, quad_kg = 0, quad_instr = 0;
    mdx::DeviceBuffer d_quad_lanes;
    // register-coefficient kernel (soap_block.hip), default options and
    // average "off" only: wavefronts (0: not used), radial groups,
    // coefficient registers, lane tables
    int block_waves = 0, block_kg = 0, block_ncr = 0;
    bool block_forced = false; // MDX_HIP_SOAP_KERNEL=block: also for inner averages of few large structures
    mdx::DeviceBuffer d_block_e1, d_block_beta, d_block_ps;
    // options beyond the GTO / uncompressed / unweighted default (mdx_soap_options)
    int Sc = 0;              // coefficient species: 1 for mu2, else S
    int compression = 0;     // 0 off, 1 mu2, 2 mu1nu1, 3 crossover
    int radial_basis = 0;    // 0 GTO, 1 polynomial
    int grid_size = 0;       // polynomial radial grid points
    int weighting = 0;       // 0 none, 1 poly, 2 pow, 3 exp
    int has_w0 = 0;
    int weighted = 0;        // any weighting function, w0 or species weight != 1
    double w_r0 = 1.0, w_c = 1.0, w_d = 0.0, w_m = 1.0, w_w0 = 1.0, eta = 0.5;
    std::vector<double> species_weights;
    mdx::DeviceBuffer d_species_w, d_poly_bw, d_poly_grid;
};

struct mdx_device_batch {
    int device = 0;
    mdx::PreparedBatch pb;
    mdx::DeviceGraph graph;
    mdx::DeviceBuffer partials;
    // Pipelined frames (mdx_hip_soap_run_frame) alternate two sets: set 0 is
    // the one above, set 1 is prepared on the first such run from the host
    // copy of the batch kept here.  A set is rebuilt only after the expansion
    // that last read it has finished (done[set]).  A frame's graph is built on
    // its set's stream (the context's graph stream for set 0, its copy stream
    // for set 1).
    std::unique_ptr<mdx::PreparedBatch> pb2;
    mdx::DeviceGraph graph2;
    mdx::DeviceBuffer partials2;
    std::vector<int32_t> host_numbers, host_pbc;
    std::vector<double> host_positions, host_cells;
    std::vector<int64_t> host_offsets;
    int next_set = 0;
    hipEvent_t ready[2] = {}; // graph of the set built (the set's frame stream)
    hipEvent_t done[2] = {};  // expansion of the set finished (main stream)
    bool queued[2] = {};      // done[set] recorded and not yet waited for
    // The last pipelined frame, whose search statistics are read (and which
    // is built and expanded again if a centre overflowed its slot) by the next
    // call on the batch: its set (-1: none), plan, output and cancel flag.
    int pending = -1;
    const mdx_soap_plan* pending_plan = nullptr;
    void* pending_out = nullptr;
    int64_t pending_pitch = 0;
    const volatile int32_t* pending_cancel = nullptr;
    ~mdx_device_batch() {
        for (int k = 0; k < 2; ++k) {
            if (queued[k]) (void)hipEventSynchronize(done[k]);
            if (ready[k] != nullptr) (void)hipEventDestroy(ready[k]);
            if (done[k] != nullptr) (void)hipEventDestroy(done[k]);
        }
    }
};

namespace mdx {
// Called after each expansion launch of an atom-level run (average off) with
// the launch's first output row and row count; the rows are written once the
// stream reaches this point.
using SliceHook = std::function<void(int64_t first_row, int64_t rows)>;

// Run the SOAP kernels (2-4) of a plan over a prepared batch whose graph is
// built; output rows x features in device memory with the given pitch.
// slice (0: the default) bounds the centres per expansion launch.
// weight_stream (pipelined frames: the stream that built the graph) takes
// the per-row weight pass of weighted plans, which then runs beside the
// previous frame's expansion; weight_ready is recorded behind it and
// stream waits for it.
void run_soap(hipStream_t stream, const mdx_soap_plan& plan, PreparedBatch& pb,
              const DeviceGraph& graph, void* out_device, int64_t pitch_bytes, DeviceBuffer& partials,
              const volatile int32_t* cancel, hipEvent_t* events, mdx_timing* timing, int64_t slice = 0,
              const SliceHook* on_slice = nullptr, hipStream_t weight_stream = nullptr,
              hipEvent_t weight_ready = nullptr);
} // namespace mdx
