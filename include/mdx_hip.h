/*
 * mdx_hip.h — C ABI of the MI355X (gfx950) SOAP library.
 *
 * This is the drop-in boundary for MDescriptor's SOAP hot path.  It carries
 * plain pointers and sizes only (no C++ or torch types), and no C++
 * exception crosses it: every entry point returns a status code and
 * mdx_hip_last_error() describes the last failure on a context.
 *
 * Each declaration names the reference interface it replaces
 * (nicheal/MDescriptor, paths relative to the repository root).
 *
 * Threading: one call at a time per context (a mutex inside the context
 * serialises callers); separate contexts are independent.  Ownership: the
 * caller owns every host buffer it passes; a context owns its device
 * buffers, its HIP stream and its pinned staging memory.
 */
#ifndef MDX_HIP_H
#define MDX_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  The Python plugin maps them onto the reference's error
 * families (src/mdescriptor/core/errors.py:215-248): OUT_OF_MEMORY ->
 * MemoryError ("backend_out_of_memory"), DEVICE_UNAVAILABLE -> ImportError
 * ("device_unavailable"), INVALID_ARGUMENT -> ValueError
 * (DescriptorInputError at the adapter), CANCELLED -> the plugin's
 * cancellation type (cpp/include/mdescriptor/detail/control.hpp:10-13). */
enum {
    MDX_OK = 0,
    MDX_INVALID_ARGUMENT = 1,
    MDX_OUT_OF_MEMORY = 2,
    MDX_DEVICE_UNAVAILABLE = 3,
    MDX_CANCELLED = 4,
    MDX_INTERNAL = 5
};

/* Flattened structure batch, the same five arrays and two counts as
 * StructureBatchView (cpp/include/mdescriptor/detail/batch.hpp:9-17):
 * numbers i32[atoms], positions f64[atoms*3] (C order), cells
 * f64[structures*9] (rows are lattice vectors), pbc i32[structures*3],
 * offsets i64[structures+1].  Pointers are host pointers. */
typedef struct mdx_batch_view {
    const int32_t* numbers;
    const double* positions;
    const double* cells;
    const int32_t* pbc;
    const int64_t* offsets;
    int64_t structures;
    int64_t atoms;
} mdx_batch_view;

/* The SoapOptions fields beyond the GTO, uncompressed, unweighted default
 * (cpp/include/mdescriptor/descriptor.hpp:17-43), filled the way
 * SoapKernel._ensure_native fills them (src/mdescriptor/descriptors/
 * _kernels/core.py:241-270).  Arrays are copied at plan creation.
 *   weighting_function: 0 none, 1 "poly", 2 "pow", 3 "exp" (soap.cpp:389-420)
 *     with r0, c, d, m; weighting_has_w0 / weighting_w0: weight of the
 *     centre's own image.
 *   species_weights: n_species values in declared order, or NULL for 1.0.
 *   compression: 0 "off", 1 "mu2", 2 "mu1nu1", 3 "crossover" (soap.cpp:373-387,
 *     933-1017).
 *   radial_basis: 0 GTO (mdx_soap_params.alphas/betas), 1 polynomial with
 *     radial_grid / radial_weights f64[grid_size] and radial_values
 *     f64[n_max * grid_size] (core.py:79-95, soap.cpp:450-492). */
typedef struct mdx_soap_options {
    int32_t weighting_function;
    int32_t weighting_has_w0;
    double weighting_r0;
    double weighting_c;
    double weighting_d;
    double weighting_m;
    double weighting_w0;
    const double* species_weights;
    int32_t compression;
    int32_t radial_basis;
    int32_t grid_size;
    const double* radial_grid;
    const double* radial_weights;
    const double* radial_values;
} mdx_soap_options;

/* SOAP parameters: SoapOptions (cpp/include/mdescriptor/descriptor.hpp:17-43).
 * alphas f64[(l_max+1)*n_max] and betas f64[(l_max+1)*n_max*n_max] (index
 * (l*n_max + n)*n_max + k) are the orthonormalised GTO basis computed by the
 * caller, exactly as the reference passes them to C++ (src/mdescriptor/
 * descriptors/_kernels/core.py:237-240) and to its CUDA plugin
 * (core.py:331-355); unused (may be NULL) with the polynomial basis.  They are
 * copied.  options may be NULL: GTO basis, compression off, no weighting,
 * unit species weights. */
typedef struct mdx_soap_params {
    const int32_t* species; /* declared order, unique, positive */
    int32_t n_species;
    int32_t n_max;
    int32_t l_max;
    double r_cut;
    double sigma;
    const double* alphas;
    const double* betas;
    int32_t average;   /* 0 "off", 1 "inner", 2 "outer" */
    int32_t out_dtype; /* bytes per output value: 4 (float32) or 8 (float64) */
    const mdx_soap_options* options;
} mdx_soap_params;

/* Per-stage device times of the last run, from HIP events recorded on the
 * context's stream around each stage. */
typedef struct mdx_timing {
    double graph_ms;     /* cell binning + neighbour count/scan/fill (kernel 1), and what the
                            expansion needs beside it (item tables; the per-row weight pass of
                            weighted plans on the register-coefficient kernel) */
    double expansion_ms; /* per-centre expansion + power spectrum + write (kernels 2-4) */
    double finalize_ms;  /* structure-level average reductions (kernel 4), 0 if off */
    double total_ms;     /* first to last event of the device pipeline */
    double h2d_ms;       /* host-to-device copies (mdx_hip_soap_compute only) */
    double d2h_ms;       /* device-to-host copy of the result (mdx_hip_soap_compute only); for
                            atom-level rows into page-locked memory, whose copy overlaps the
                            expansion launches, only the part left after the last kernel */
    int64_t pairs;       /* neighbour pairs found at the padded SOAP cutoff */
    int64_t binned;      /* periodic images binned into the cell grid */
    int64_t expansion_launches; /* launches of the expansion kernel in the run */
    int64_t expansion_tiles;    /* 16x16 tiles of the matrix-core kernel's template;
                                   minus the wavefronts of the 4x4-block kernel
                                   when that ran; -(1000 + wavefronts) when the
                                   register-coefficient kernel ran; 0 when the
                                   generic kernel ran */
} mdx_timing;

typedef struct mdx_hip_ctx mdx_hip_ctx;
typedef struct mdx_soap_plan mdx_soap_plan;
typedef struct mdx_device_batch mdx_device_batch;

/* Context on one HIP device: stream, device arena, pinned staging.
 * Replaces CudaExecutionContext (cpp/cuda/include/mdescriptor/cuda/context.hpp:27-78)
 * and the lazy device selection of Backend (cpp/cuda/src/backend.cu:338-356). */
int mdx_hip_create(int device, mdx_hip_ctx** out);
void mdx_hip_destroy(mdx_hip_ctx* ctx);

/* Last error message on this context ("" when none).  Replaces the
 * exception text of check_cuda (cpp/cuda/include/mdescriptor/cuda/error.hpp:15-30). */
const char* mdx_hip_last_error(const mdx_hip_ctx* ctx);

/* Validated, device-resident SOAP plan (prefactors, beta, feature table).
 * Replaces SoapCalculator(SoapOptions) + prepare_soap
 * (cpp/src/standalone/soap.cpp:507-572, 1248) and the CUDA payload upload
 * (cpp/cuda/src/extended_descriptors_soap.cuh:898-906).  *features receives
 * the feature count (soap.cpp:373-387). */
int mdx_hip_soap_plan_create(mdx_hip_ctx* ctx, const mdx_soap_params* params, mdx_soap_plan** out,
                             int64_t* features);
void mdx_hip_soap_plan_destroy(mdx_soap_plan* plan);

/* Rows of the result for this plan and batch: structures when averaging,
 * else atoms (soap.cpp:1216-1217, 1240-1243). */
int64_t mdx_hip_soap_rows(const mdx_soap_plan* plan, const mdx_batch_view* batch);

/* Full compute: validate, upload, run, download into out_host
 * (rows x features values of out_dtype, row stride out_pitch_bytes).
 * With average "off" and out_host in page-locked memory (mdx_hip_host_alloc)
 * the expansion runs in about eight launches and each launch's rows are
 * copied out on a second stream while the next ones compute.
 * Replaces SoapCalculator::compute (soap.cpp:1254-1258) as called through
 * compute_soap_array (cpp/src/bindings/module.cpp:431-452), and the CUDA
 * Backend::compute SOAP path (cpp/cuda/src/backend.cu:338-631 ->
 * extended_descriptors_soap.cuh:799-1125).  cancel_flag (nullable) is polled
 * between stages and launches; a non-zero value returns MDX_CANCELLED.
 * timing (nullable) receives the stage times. */
int mdx_hip_soap_compute(mdx_hip_ctx* ctx, const mdx_soap_plan* plan, const mdx_batch_view* batch,
                         void* out_host, int64_t out_rows, int64_t out_pitch_bytes,
                         const volatile int32_t* cancel_flag, mdx_timing* timing);

/* Device-resident path: upload and prepare a batch once ...
 * (the H2D part of Backend::compute, cpp/cuda/src/backend.cu:353-356) */
int mdx_hip_batch_upload(mdx_hip_ctx* ctx, const mdx_soap_plan* plan, const mdx_batch_view* batch,
                         mdx_device_batch** out);
void mdx_hip_batch_destroy(mdx_device_batch* batch);

/* New positions for a device-resident batch (a new frame of the same system:
 * numbers, cells, pbc and offsets are kept): positions f64[atoms*3], C order,
 * in host or device memory.  Replaces the position part of the per-call
 * upload of Backend::compute (cpp/cuda/src/backend.cu:353-356) for a caller
 * that keeps its batch on the device; the reference itself takes each frame
 * as a new StructureBatch (src/mdescriptor/core/input.py:39-122).  Everything
 * that depends on positions (cell grid, regions of interest, home cells,
 * graph) is rebuilt on the device by the next run, as compute_soap rebuilds
 * its grid on every call (cpp/src/standalone/soap.cpp:1218-1245,
 * cpp/src/common/neighbor.cpp:135-194, 551).  Host positions are checked
 * ("positions must be finite") and copied before the call returns.  Device
 * positions are copied on the context's stream, after the work already
 * queued there and before the next run on this context reads them; the caller
 * keeps them unchanged until that run returns.  A non-finite device position
 * makes that run return MDX_INVALID_ARGUMENT with the same message. */
int mdx_hip_batch_set_positions(mdx_hip_ctx* ctx, mdx_device_batch* batch, const double* positions);

/* ... then run the SOAP pipeline on it, writing into device memory out_device
 * (rows x features, row stride out_pitch_bytes).  No host copy of the result;
 * the call returns after the stream has finished.  Same computation as
 * mdx_hip_soap_compute. */
int mdx_hip_soap_run(mdx_hip_ctx* ctx, const mdx_soap_plan* plan, mdx_device_batch* batch,
                     void* out_device, int64_t out_pitch_bytes, const volatile int32_t* cancel_flag,
                     mdx_timing* timing);

/* Size of the static device scratch array of mdx_hip_soap_run_noalloc. */
#define MDX_NOALLOC_SCRATCH_BYTES (64u << 20)

/* mdx_hip_soap_run without device allocation.  No counterpart in the
 * reference: for callers that cannot allocate device memory during the run
 * (tight serving loops, code that must not call hipMalloc).  Same arguments,
 * kernels and results as mdx_hip_soap_run; the run's scratch (neighbour graph,
 * partial sums of the averaged modes) lives in one static device array of
 * MDX_NOALLOC_SCRATCH_BYTES per device instead of buffers owned by the batch.
 * The plan, the batch and out_device are the caller's, made beforehand.  A
 * batch whose scratch does not fit returns MDX_INVALID_ARGUMENT with a message
 * that names the maximum.  All contexts on one device share its array, which
 * keeps the last call's contents: calls that overlap on one device (through
 * different contexts; one context serialises its own calls) race.  Frames
 * still queued on the batch by mdx_hip_soap_run_frame are settled first, as
 * by mdx_hip_batch_wait, which allocates if one of them overflowed its slot:
 * call mdx_hip_batch_wait beforehand to keep the call itself free of
 * allocation. */
int mdx_hip_soap_run_noalloc(mdx_hip_ctx* ctx, const mdx_soap_plan* plan, mdx_device_batch* batch,
                             void* out_device, int64_t out_pitch_bytes, const volatile int32_t* cancel_flag,
                             mdx_timing* timing);

/* A trajectory frame on a device-resident batch without waiting for it:
 * positions (f64[atoms*3], C order, host or device memory) replace the
 * batch's, and the SOAP pipeline runs on them into out_device, as
 * mdx_hip_batch_set_positions followed by mdx_hip_soap_run.  No counterpart
 * in the reference, which rebuilds its grid and graph in each compute_soap
 * call and returns after the call (cpp/src/standalone/soap.cpp:1218-1245):
 * for callers that step through frames (molecular dynamics, trajectory
 * analysis).  The call returns once the frame's graph search and expansion
 * are queued; the positions have been read by then.  The batch alternates
 * two sets of device buffers, each with its own stream for the graph, so the
 * graph of one frame is built while the previous frame's search and
 * expansion run.  A frame's search statistics are read by the next call on
 * the batch (this one or mdx_hip_batch_wait): a centre that overflowed its
 * slot has that frame built and expanded again before any later frame's
 * expansion.  Results are bit-identical to the synchronous run.  A frame's
 * out_device is complete after mdx_hip_batch_wait on the batch (or after a
 * later synchronous call on it); the caller keeps the output, the plan and
 * the cancel flag alive until then, and reads the output only then.  A
 * non-finite position returns MDX_INVALID_ARGUMENT ("positions must be
 * finite"); the frames before it are unaffected. */
int mdx_hip_soap_run_frame(mdx_hip_ctx* ctx, const mdx_soap_plan* plan, mdx_device_batch* batch,
                           const double* positions, void* out_device, int64_t out_pitch_bytes,
                           const volatile int32_t* cancel_flag);

/* Settle and wait for every frame queued on the batch by
 * mdx_hip_soap_run_frame. */
int mdx_hip_batch_wait(mdx_hip_ctx* ctx, mdx_device_batch* batch);

/* Neighbour graph on the device, for parity and the pair-level API.
 * Replaces build_neighbor_graph (cpp/src/common/neighbor.cpp:703-768) as
 * exported by _native.build_neighbor_graph (cpp/src/bindings/module.cpp:887-935):
 * CSR over all atoms of the batch, rows in the reference's candidate order,
 * atom indices global to the batch, self pair and periodic self-images
 * included, boundary inclusive when include_boundary != 0.
 * mdx_hip_neighbors_build computes and keeps the graph on the context and
 * returns its pair count; mdx_hip_neighbors_fetch copies it out into caller
 * buffers: offsets i64[atoms+1], neighbors i32[pairs], shifts i32[pairs*3],
 * displacements f64[pairs*3], distance2 f64[pairs] (any may be NULL). */
int mdx_hip_neighbors_build(mdx_hip_ctx* ctx, const mdx_batch_view* batch, double cutoff,
                            int32_t include_boundary, int64_t* pairs);
int mdx_hip_neighbors_fetch(mdx_hip_ctx* ctx, int64_t* offsets, int32_t* neighbors, int32_t* shifts,
                            double* displacements, double* distance2);

/* NeighborList descriptor on the device.  Replaces compute_neighbor_list
 * (cpp/src/standalone/neighbor_list.cpp:15-78; declared in
 * cpp/include/mdescriptor/local_descriptors.hpp:54-60) as bound by
 * _cpp.compute_neighbor_list (cpp/src/bindings/module.cpp:772-798, 1012) and
 * the CUDA plugin's NeighborList branch (cpp/cuda/src/backend.cu:358-471).
 * Every centre's pairs within cutoff (boundary inclusive), in the
 * reference's order, centre-major over the batch; the exact self pair (same
 * atom, zero shift) is dropped unless self_pairs != 0, and with
 * full_neighbor_list == 0 only the orientation kept by keep_half_neighbor
 * (cpp/include/mdescriptor/detail/neighbor_filter.hpp:18-38) remains.
 * mdx_hip_neighbor_list computes the list on the device, keeps it on the
 * context and returns its pair count in *pairs; cancel_flag as for
 * mdx_hip_soap_compute.  A non-finite or non-positive cutoff is rejected with
 * the reference's message. */
int mdx_hip_neighbor_list(mdx_hip_ctx* ctx, const mdx_batch_view* batch, double cutoff, int32_t full_neighbor_list,
                          int32_t self_pairs, const volatile int32_t* cancel_flag, int64_t* pairs);

/* Writes the last neighbour list of the context.  Any pointer may be NULL
 * (that output is skipped) and each may be host or device memory (device
 * memory aligned to 8 bytes is written in place by the kernel; other
 * destinations receive a copy):
 *   table   f64[pairs*9]  DescriptorPairTable rows (local_descriptors.hpp:29-34):
 *                         centre, neighbour (global atom indices), cell
 *                         shifts a b c, dx dy dz, distance
 *   values  f64[pairs*4]  dx dy dz distance, the public result's values
 *                         (src/mdescriptor/descriptors/_kernels/local.py:98-110)
 *   samples i64[pairs*6]  structure, local centre, local neighbour, shifts
 *                         a b c (pair_samples, src/mdescriptor/core/result.py:257-300)
 *   offsets i64[structures+1]  first pair of each structure
 *                         (DescriptorPairTable::offsets). */
int mdx_hip_neighbor_list_fetch(mdx_hip_ctx* ctx, double* table, double* values, int64_t* samples,
                                int64_t* offsets);

/* Device stage times of the last neighbour list on the context, from HIP
 * events on its stream: the graph (kernel 1), the keep-count and its scan,
 * and the record fill of the last fetch (0 before a fetch).  A diagnostic
 * without reference counterpart, like mdx_timing. */
typedef struct mdx_list_timing {
    double graph_ms;
    double count_ms;
    double fill_ms;
    int64_t graph_pairs; /* pairs of the graph before the filter */
    int64_t pairs;       /* kept pairs */
    int64_t binned;      /* periodic images binned into the cell grid */
} mdx_list_timing;
int mdx_hip_neighbor_list_timing(mdx_hip_ctx* ctx, mdx_list_timing* timing);

/* Page-locked host memory for result matrices.  mdx_hip_soap_compute copies
 * into such a buffer with one DMA at the full PCIe rate; into pageable memory
 * it stages through the context's pinned ring and copies out on host threads.
 * No reference counterpart: the reference's CUDA context copies straight into
 * the caller's pageable buffer (download_output_slice_into,
 * cpp/cuda/src/context.cu:115-137).  Returns MDX_OUT_OF_MEMORY when it cannot
 * allocate. */
int mdx_hip_host_alloc(size_t bytes, void** out);
void mdx_hip_host_free(void* ptr);

/* Library version and build target, for diagnostics. */
const char* mdx_hip_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MDX_HIP_H */
