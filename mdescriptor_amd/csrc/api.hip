// The extern "C" boundary of the SOAP library (declared in include/mdx_hip.h).
//
// Everything below the boundary throws mdx::Error; every entry point catches
// and returns a status code, keeping the message on the context.  Calls on
// one context are serialised by its mutex (the reference serialises a
// calculator the same way, cpp/src/standalone/soap.cpp:1255 and
// cpp/cuda/src/backend.cu:339-345).
#include "mdx_internal.h"
#include "soap_mfma.h"
#include "soap_block.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <new>
#include <thread>
#include <unordered_set>

namespace {

thread_local std::string g_last_error;

// Device scratch of mdx_hip_soap_run_noalloc: the neighbour graph and the
// partial sums of one run.  Every device that loads the library holds one
// copy until the process ends.  Host code never names the array itself (its
// host-side symbol is not a device address): it uses the device address that
// hipGetSymbolAddress returns, looked up once per device at context creation.
constexpr size_t kStaticScratchBytes = size_t(MDX_NOALLOC_SCRATCH_BYTES);
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

// Device address of `scratch` on the current device (device index < 64).
char* static_scratch(int device) {
    static std::mutex lock;
    static char* address[64] = {};
    if (device < 0 || device >= 64) throw mdx::Error(MDX_INVALID_ARGUMENT, "HIP device index out of range");
    std::lock_guard<std::mutex> guard(lock);
    if (address[device] == nullptr) {
        void* p = nullptr;
        MDX_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (p == nullptr) throw mdx::Error(MDX_INTERNAL, "no device address for the static scratch array");
        address[device] = static_cast<char*>(p);
    }
    return address[device];
}

template <typename Fn>
int guarded(mdx_hip_ctx* ctx, Fn&& fn) {
    std::string message;
    int status = MDX_OK;
    try {
        fn();
    } catch (const mdx::Error& e) {
        status = e.status;
        message = e.what();
    } catch (const std::bad_alloc&) {
        status = MDX_OUT_OF_MEMORY;
        message = "host out of memory";
    } catch (const std::exception& e) {
        status = MDX_INTERNAL;
        message = e.what();
    } catch (...) {
        status = MDX_INTERNAL;
        message = "unknown error";
    }
    if (ctx != nullptr) ctx->last_error = message;
    g_last_error = message;
    return status;
}

struct DeviceScope {
    int previous = -1;
    explicit DeviceScope(int device) {
        if (hipGetDevice(&previous) != hipSuccess) previous = -1;
        MDX_HIP(hipSetDevice(device));
    }
    ~DeviceScope() {
        if (previous >= 0) (void)hipSetDevice(previous);
    }
};

float elapsed(hipEvent_t a, hipEvent_t b) {
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, a, b) != hipSuccess) return 0.0f;
    return ms;
}

void check_cancel(const volatile int32_t* cancel) {
    if (cancel != nullptr && *cancel != 0) throw mdx::Error(MDX_CANCELLED, "descriptor computation was cancelled");
}

// Pair export for the neighbour API: one thread per pair.
__global__ void k_export_pairs(const int64_t* pair_start, int64_t atoms, int64_t pairs, const uint32_t* pair_bin,
                               const double* positions, const double* bx, const double* by, const double* bz,
                               const int32_t* batom, const int32_t* bimage, const mdx::ImageDesc* images,
                               int32_t* out_atoms, int32_t* out_shifts, double* out_disp, double* out_d2) {
    for (int64_t p = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; p < pairs;
         p += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        int64_t lo = 0, hi = atoms;
        while (hi - lo > 1) {
            const int64_t mid = (lo + hi) / 2;
            if (pair_start[mid] <= p) lo = mid; else hi = mid;
        }
        while (lo + 1 < atoms && pair_start[lo + 1] <= p) ++lo;
        const uint32_t b = pair_bin[p];
        const double dx = bx[b] - positions[lo * 3 + 0];
        const double dy = by[b] - positions[lo * 3 + 1];
        const double dz = bz[b] - positions[lo * 3 + 2];
        out_atoms[p] = batom[b];
        const mdx::ImageDesc& im = images[bimage[b]];
        out_shifts[p * 3 + 0] = im.n[0];
        out_shifts[p * 3 + 1] = im.n[1];
        out_shifts[p * 3 + 2] = im.n[2];
        out_disp[p * 3 + 0] = dx;
        out_disp[p * 3 + 1] = dy;
        out_disp[p * 3 + 2] = dz;
        out_d2[p] = dx * dx + dy * dy + dz * dz;
    }
}

double soap_padding(double sigma) {
    // graph cutoff padding, cpp/src/standalone/soap.cpp:1214
    return sigma * std::sqrt(-2.0 * std::log(1e-3));
}

void validate_params(const mdx_soap_params& p) {
    if (p.species == nullptr || p.n_species < 1) throw mdx::Error(MDX_INVALID_ARGUMENT, "species must not be empty");
    if (p.n_species > mdx::kMaxSpecies) {
        throw mdx::Error(MDX_INVALID_ARGUMENT, "the HIP SOAP backend supports at most 16 species");
    }
    std::unordered_set<int32_t> seen;
    for (int t = 0; t < p.n_species; ++t) {
        if (p.species[t] <= 0) throw mdx::Error(MDX_INVALID_ARGUMENT, "species must contain positive atomic numbers");
        if (!seen.insert(p.species[t]).second) {
            throw mdx::Error(MDX_INVALID_ARGUMENT, "species must contain unique atomic numbers");
        }
    }
    // soap.cpp:1152-1158
    if (!std::isfinite(p.r_cut) || !std::isfinite(p.sigma) || p.r_cut <= 0.0 || p.sigma <= 0.0 || p.n_max < 1
        || p.l_max < 0 || p.l_max > mdx::kMaxLmax || p.average < 0 || p.average > 2
        || (p.out_dtype != 4 && p.out_dtype != 8)) {
        throw mdx::Error(MDX_INVALID_ARGUMENT, "invalid SOAP parameters");
    }
    if (p.n_max > mdx::kMaxNmax) {
        throw mdx::Error(MDX_INVALID_ARGUMENT, "the HIP SOAP backend supports n_max <= 16");
    }
    const mdx_soap_options* o = p.options;
    if (o != nullptr && (o->radial_basis < 0 || o->radial_basis > 1 || o->compression < 0 || o->compression > 3)) {
        throw mdx::Error(MDX_INVALID_ARGUMENT, "invalid SOAP parameters");
    }
    const bool polynomial = o != nullptr && o->radial_basis == 1;
    const int L = p.l_max + 1;
    // soap.cpp:1160-1209, in its order
    if (!polynomial) {
        if (p.alphas == nullptr || p.betas == nullptr) {
            throw mdx::Error(MDX_INVALID_ARGUMENT, "invalid SOAP radial basis size");
        }
        for (int i = 0; i < L * p.n_max; ++i) {
            if (!std::isfinite(p.alphas[i])) throw mdx::Error(MDX_INVALID_ARGUMENT, "SOAP radial basis must be finite");
        }
        for (int i = 0; i < L * p.n_max * p.n_max; ++i) {
            if (!std::isfinite(p.betas[i])) throw mdx::Error(MDX_INVALID_ARGUMENT, "SOAP radial basis must be finite");
        }
    } else {
        if (o->grid_size < 2 || o->radial_grid == nullptr || o->radial_weights == nullptr
            || o->radial_values == nullptr) {
            throw mdx::Error(MDX_INVALID_ARGUMENT, "invalid SOAP polynomial radial basis size");
        }
        if (o->grid_size > 4096) {
            throw mdx::Error(MDX_INVALID_ARGUMENT, "the HIP SOAP backend supports at most 4096 radial grid points");
        }
        for (int q = 0; q < o->grid_size; ++q) {
            if (!std::isfinite(o->radial_grid[q]) || o->radial_grid[q] < 0.0 || o->radial_grid[q] > p.r_cut) {
                throw mdx::Error(MDX_INVALID_ARGUMENT, "SOAP polynomial radial grid must be finite and in range");
            }
        }
        for (int q = 0; q < o->grid_size; ++q) {
            if (!std::isfinite(o->radial_weights[q]) || o->radial_weights[q] <= 0.0) {
                throw mdx::Error(MDX_INVALID_ARGUMENT, "SOAP polynomial radial weights must be positive and finite");
            }
        }
        for (int64_t i = 0; i < static_cast<int64_t>(o->grid_size) * p.n_max; ++i) {
            if (!std::isfinite(o->radial_values[i])) {
                throw mdx::Error(MDX_INVALID_ARGUMENT, "SOAP polynomial radial basis must be finite");
            }
        }
    }
    if (o != nullptr && o->species_weights != nullptr) {
        for (int t = 0; t < p.n_species; ++t) {
            if (!std::isfinite(o->species_weights[t])) {
                throw mdx::Error(MDX_INVALID_ARGUMENT, "SOAP species weights must be finite");
            }
        }
    }
    if (o != nullptr && o->weighting_function != 0) {
        if (o->weighting_function < 1 || o->weighting_function > 3 || !std::isfinite(o->weighting_r0)
            || o->weighting_r0 <= 0.0 || !std::isfinite(o->weighting_c) || o->weighting_c < 0.0
            || !std::isfinite(o->weighting_d) || o->weighting_d < 0.0 || !std::isfinite(o->weighting_m)
            || o->weighting_m < 0.0) {
            throw mdx::Error(MDX_INVALID_ARGUMENT, "invalid SOAP weighting parameters");
        }
    }
    if (o != nullptr && o->weighting_has_w0 && (!std::isfinite(o->weighting_w0) || o->weighting_w0 < 0.0)) {
        throw mdx::Error(MDX_INVALID_ARGUMENT, "invalid SOAP w0 weighting");
    }
    const int64_t coeff = static_cast<int64_t>(p.n_species) * p.n_max * L * L;
    if (coeff * 8 > 96 * 1024) {
        throw mdx::Error(MDX_INVALID_ARGUMENT,
                         "SOAP shape exceeds the HIP backend coefficient budget (species*n_max*(l_max+1)^2 <= 12288)");
    }
}

template <typename T>
void upload(mdx::DeviceBuffer& buf, const std::vector<T>& host) {
    buf.reserve(std::max<size_t>(1, host.size() * sizeof(T)));
    if (!host.empty()) MDX_HIP(hipMemcpy(buf.ptr, host.data(), host.size() * sizeof(T), hipMemcpyHostToDevice));
}

void fill_timing(mdx_hip_ctx* ctx, mdx_timing* timing, bool with_copies) {
    if (timing == nullptr) return;
    hipEvent_t* ev = ctx->events;
    // the graph and what the expansion needs beside it (item tables, the
    // weighted modes' per-row weights)
    timing->graph_ms = elapsed(ev[0], ev[2]);
    timing->expansion_ms = elapsed(ev[2], ev[3]);
    timing->finalize_ms = elapsed(ev[3], ev[4]);
    timing->total_ms = elapsed(ev[0], ev[4]);
    if (with_copies) {
        timing->h2d_ms = elapsed(ev[5], ev[0]);
        timing->d2h_ms = elapsed(ev[4], ev[6]);
    } else {
        timing->h2d_ms = 0.0;
        timing->d2h_ms = 0.0;
    }
}

void run_pipeline(mdx_hip_ctx* ctx, const mdx_soap_plan& plan, mdx::PreparedBatch& pb, mdx::DeviceGraph& graph,
                  mdx::DeviceBuffer& partials, void* out_device, int64_t pitch, const volatile int32_t* cancel,
                  mdx_timing* timing, int64_t slice = 0, const mdx::SliceHook* on_slice = nullptr) {
    hipStream_t s = ctx->stream;
    MDX_HIP(hipEventRecord(ctx->events[0], s));
    // the expansion is queued behind the slotted search without waiting for
    // its statistics (no host round trip between them); they are checked
    // after, and a batch whose centre overflowed its slot runs again on the
    // compact layout
    mdx::build_graph(s, pb, graph, cancel, true, true);
    MDX_HIP(hipEventRecord(ctx->events[1], s));
    check_cancel(cancel);
    mdx::run_soap(s, plan, pb, graph, out_device, pitch, partials, cancel, ctx->events, timing, slice, on_slice);
    if (!mdx::complete_graph(pb, graph, cancel)) {
        MDX_HIP(hipStreamSynchronize(s)); // the first expansion's buffers are replaced
        mdx::build_graph(s, pb, graph, cancel, true, false, true);
        MDX_HIP(hipEventRecord(ctx->events[1], s));
        check_cancel(cancel);
        mdx::run_soap(s, plan, pb, graph, out_device, pitch, partials, cancel, ctx->events, timing, slice, on_slice);
    }
    const int64_t pairs = graph.pairs;
    const int64_t rows = plan.average != 0 ? pb.structures : pb.atoms;
    if (rows == 0 || plan.features == 0) {
        MDX_HIP(hipEventRecord(ctx->events[2], s));
        MDX_HIP(hipEventRecord(ctx->events[3], s));
        MDX_HIP(hipEventRecord(ctx->events[4], s));
    }
    if (timing != nullptr) {
        timing->pairs = pairs;
        timing->binned = graph.binned;
    }
}

// True for memory from hipHostMalloc (page-locked, DMA-able at full PCIe
// rate); pageable memory reports "unregistered" or an error, which is cleared.
bool is_pinned_host(const void* p) {
    hipPointerAttribute_t attr{};
    const hipError_t rc = hipPointerGetAttributes(&attr, p);
    if (rc != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeHost;
}

// True for device memory (hipMalloc and the like), which kernels may write
// directly.
bool is_device_memory(const void* p) {
    hipPointerAttribute_t attr{};
    const hipError_t rc = hipPointerGetAttributes(&attr, p);
    if (rc != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice;
}

// Copy rows x row_bytes of device memory into the caller's host rows (row
// stride pitch) and wait for it.  Pinned destinations take one DMA.  Pageable
// ones go through the context's pinned staging ring in chunks of whole rows:
// while the DMA fills one half of the ring, host threads copy the other half
// out, so the transfer runs near the PCIe rate instead of the driver's
// pageable path (which the reference's download_output_slice_into,
// cpp/cuda/src/context.cu:115-137, takes with one plain copy).
void download_result(mdx_hip_ctx* ctx, const void* src, int64_t rows, int64_t row_bytes, void* dst, int64_t pitch) {
    hipStream_t s = ctx->stream;
    if (rows <= 0 || row_bytes <= 0) return;
    const size_t total = static_cast<size_t>(rows) * static_cast<size_t>(row_bytes);
    if (is_pinned_host(dst)) {
        if (pitch == row_bytes) {
            MDX_HIP(hipMemcpyAsync(dst, src, total, hipMemcpyDeviceToHost, s));
        } else {
            MDX_HIP(hipMemcpy2DAsync(dst, static_cast<size_t>(pitch), src, static_cast<size_t>(row_bytes),
                                     static_cast<size_t>(row_bytes), static_cast<size_t>(rows), hipMemcpyDeviceToHost,
                                     s));
        }
        MDX_HIP(hipStreamSynchronize(s));
        return;
    }
    constexpr size_t kStageHalf = size_t(64) << 20;
    const int64_t chunk_rows = std::max<int64_t>(1, static_cast<int64_t>(kStageHalf / static_cast<size_t>(row_bytes)));
    const size_t half = static_cast<size_t>(chunk_rows) * static_cast<size_t>(row_bytes);
    if (ctx->pinned == nullptr || ctx->pinned_bytes < 2 * half) {
        if (ctx->pinned != nullptr) (void)hipHostFree(ctx->pinned);
        ctx->pinned = nullptr;
        ctx->pinned_bytes = 0;
        const hipError_t rc = hipHostMalloc(&ctx->pinned, 2 * half, hipHostMallocDefault);
        if (rc != hipSuccess || ctx->pinned == nullptr) {
            (void)hipGetLastError();
            ctx->pinned = nullptr;
            throw mdx::Error(MDX_OUT_OF_MEMORY, "cannot allocate pinned staging for the result download");
        }
        ctx->pinned_bytes = 2 * half;
    }
    char* ring[2] = {static_cast<char*>(ctx->pinned), static_cast<char*>(ctx->pinned) + half};
    const int64_t chunks = (rows + chunk_rows - 1) / chunk_rows;
    auto enqueue = [&](int64_t c) {
        const int64_t r0 = c * chunk_rows;
        const int64_t nr = std::min(chunk_rows, rows - r0);
        MDX_HIP(hipMemcpyAsync(ring[c & 1], static_cast<const char*>(src) + r0 * row_bytes,
                               static_cast<size_t>(nr) * static_cast<size_t>(row_bytes), hipMemcpyDeviceToHost, s));
        MDX_HIP(hipEventRecord(ctx->stage_events[c & 1], s));
    };
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const int threads = static_cast<int>(std::min(8u, hw));
    enqueue(0);
    for (int64_t c = 0; c < chunks; ++c) {
        // the other half was copied out in the previous iteration, so it can take the next DMA
        if (c + 1 < chunks) enqueue(c + 1);
        MDX_HIP(hipEventSynchronize(ctx->stage_events[c & 1]));
        const int64_t r0 = c * chunk_rows;
        const int64_t nr = std::min(chunk_rows, rows - r0);
        const char* from = ring[c & 1];
        char* to = static_cast<char*>(dst) + r0 * pitch;
        auto copy_rows = [&](int64_t a, int64_t b) {
            if (pitch == row_bytes) {
                std::memcpy(to + a * row_bytes, from + a * row_bytes, static_cast<size_t>((b - a) * row_bytes));
            } else {
                for (int64_t r = a; r < b; ++r) {
                    std::memcpy(to + r * pitch, from + r * row_bytes, static_cast<size_t>(row_bytes));
                }
            }
        };
        const int parts = static_cast<int>(std::min<int64_t>(threads, nr));
        if (parts <= 1) {
            copy_rows(0, nr);
            continue;
        }
        std::vector<std::thread> pool;
        pool.reserve(static_cast<size_t>(parts - 1));
        for (int t = 1; t < parts; ++t) {
            pool.emplace_back(copy_rows, nr * t / parts, nr * (t + 1) / parts);
        }
        copy_rows(0, nr / parts);
        for (auto& th : pool) th.join();
    }
}

} // namespace

extern "C" {

int mdx_hip_host_alloc(size_t bytes, void** out) {
    if (out == nullptr) return MDX_INVALID_ARGUMENT;
    *out = nullptr;
    return guarded(nullptr, [&] {
        void* p = nullptr;
        const hipError_t rc = hipHostMalloc(&p, std::max<size_t>(1, bytes), hipHostMallocDefault);
        if (rc != hipSuccess || p == nullptr) {
            (void)hipGetLastError();
            throw mdx::Error(MDX_OUT_OF_MEMORY, "cannot allocate pinned host memory");
        }
        *out = p;
    });
}

void mdx_hip_host_free(void* p) {
    if (p != nullptr) (void)hipHostFree(p);
}

const char* mdx_hip_version(void) { return "mdx_hip 0.2.0 (gfx950)"; }

const char* mdx_hip_last_error(const mdx_hip_ctx* ctx) {
    return ctx != nullptr ? ctx->last_error.c_str() : g_last_error.c_str();
}

int mdx_hip_create(int device, mdx_hip_ctx** out) {
    if (out == nullptr) return MDX_INVALID_ARGUMENT;
    *out = nullptr;
    return guarded(nullptr, [&] {
        int count = 0;
        const hipError_t rc = hipGetDeviceCount(&count);
        if (rc != hipSuccess || count <= 0) {
            throw mdx::Error(MDX_DEVICE_UNAVAILABLE, "no HIP device is available");
        }
        if (device < 0 || device >= count) throw mdx::Error(MDX_INVALID_ARGUMENT, "HIP device index out of range");
        auto ctx = new mdx_hip_ctx();
        try {
            DeviceScope scope(device);
            ctx->device = device;
            MDX_HIP(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking));
            MDX_HIP(hipStreamCreateWithFlags(&ctx->copy_stream, hipStreamNonBlocking));
            MDX_HIP(hipStreamCreateWithFlags(&ctx->graph_stream, hipStreamNonBlocking));
            for (auto& ev : ctx->events) MDX_HIP(hipEventCreate(&ev));
            for (auto& ev : ctx->stage_events) MDX_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
            for (auto& ev : ctx->list_events) MDX_HIP(hipEventCreate(&ev));
            ctx->finished.prepare();
            // what mdx_hip_soap_run_noalloc needs beyond the scratch array:
            // the pinned statistics words and the read-back event
            ctx->arena.base = static_scratch(device);
            ctx->arena.capacity = kStaticScratchBytes;
            ctx->static_graph.for_each_buffer([&](mdx::DeviceBuffer& b) { b.arena = &ctx->arena; });
            ctx->static_partials.arena = &ctx->arena;
            ctx->static_graph.stats_host.get(mdx::kStatWords);
            ctx->static_graph.read_back.prepare();
        } catch (...) {
            mdx_hip_destroy(ctx);
            throw;
        }
        *out = ctx;
    });
}

void mdx_hip_destroy(mdx_hip_ctx* ctx) {
    if (ctx == nullptr) return;
    int previous = -1;
    (void)hipGetDevice(&previous);
    (void)hipSetDevice(ctx->device);
    {
        std::lock_guard<std::mutex> lock(ctx->mutex);
        if (ctx->stream != nullptr) (void)hipStreamSynchronize(ctx->stream);
        if (ctx->copy_stream != nullptr) (void)hipStreamSynchronize(ctx->copy_stream);
        if (ctx->graph_stream != nullptr) (void)hipStreamSynchronize(ctx->graph_stream);
        for (auto& ev : ctx->slice_events) {
            if (ev != nullptr) (void)hipEventDestroy(ev);
        }
        ctx->slice_events.clear();
        for (auto& ev : ctx->events) {
            if (ev != nullptr) (void)hipEventDestroy(ev);
            ev = nullptr;
        }
        for (auto& ev : ctx->stage_events) {
            if (ev != nullptr) (void)hipEventDestroy(ev);
            ev = nullptr;
        }
        for (auto& ev : ctx->list_events) {
            if (ev != nullptr) (void)hipEventDestroy(ev);
            ev = nullptr;
        }
        if (ctx->pinned != nullptr) (void)hipHostFree(ctx->pinned);
        ctx->pinned = nullptr;
    }
    hipStream_t stream = ctx->stream;
    hipStream_t copy_stream = ctx->copy_stream;
    hipStream_t graph_stream = ctx->graph_stream;
    delete ctx; // device buffers are freed by their destructors
    if (stream != nullptr) (void)hipStreamDestroy(stream);
    if (copy_stream != nullptr) (void)hipStreamDestroy(copy_stream);
    if (graph_stream != nullptr) (void)hipStreamDestroy(graph_stream);
    if (previous >= 0) (void)hipSetDevice(previous);
}

int mdx_hip_soap_plan_create(mdx_hip_ctx* ctx, const mdx_soap_params* params, mdx_soap_plan** out,
                             int64_t* features) {
    if (ctx == nullptr || params == nullptr || out == nullptr) return MDX_INVALID_ARGUMENT;
    *out = nullptr;
    std::lock_guard<std::mutex> lock(ctx->mutex);
    return guarded(ctx, [&] {
        const mdx_soap_params& p = *params;
        validate_params(p);
        DeviceScope scope(ctx->device);
        auto plan = new mdx_soap_plan();
        try {
            plan->device = ctx->device;
            plan->S = p.n_species;
            plan->n = p.n_max;
            plan->l_max = p.l_max;
            plan->L = p.l_max + 1;
            plan->H = plan->L * plan->L;
            plan->LN = plan->L * p.n_max;
            plan->average = p.average;
            plan->out_dtype = p.out_dtype;
            plan->r_cut = p.r_cut;
            plan->sigma = p.sigma;
            plan->cutoff = p.r_cut + soap_padding(p.sigma);
            plan->species.assign(p.species, p.species + p.n_species);
            const mdx_soap_options* o = p.options;
            plan->compression = o != nullptr ? o->compression : 0;
            plan->radial_basis = o != nullptr ? o->radial_basis : 0;
            plan->weighting = o != nullptr ? o->weighting_function : 0;
            plan->has_w0 = o != nullptr && o->weighting_has_w0 ? 1 : 0;
            if (o != nullptr) {
                plan->w_r0 = o->weighting_r0;
                plan->w_c = o->weighting_c;
                plan->w_d = o->weighting_d;
                plan->w_m = o->weighting_m;
                plan->w_w0 = o->weighting_w0;
            }
            plan->species_weights.assign(static_cast<size_t>(plan->S), 1.0);
            if (o != nullptr && o->species_weights != nullptr) {
                plan->species_weights.assign(o->species_weights, o->species_weights + plan->S);
            }
            bool unit_species = true;
            for (double v : plan->species_weights) unit_species = unit_species && v == 1.0;
            plan->weighted = plan->weighting != 0 || plan->has_w0 || !unit_species ? 1 : 0;
            // coefficient species: mu2 sums every neighbour into one density (soap.cpp:710)
            plan->Sc = plan->compression == 1 ? 1 : plan->S;
            {
                // soap_features, soap.cpp:373-387
                const int64_t S = plan->S, n = plan->n, Lw = plan->L;
                switch (plan->compression) {
                case 1: plan->features = n * (n + 1) / 2 * Lw; break;
                case 2: plan->features = S * n * n * Lw; break;
                case 3: plan->features = S * n * (n + 1) / 2 * Lw; break;
                default: plan->features = S * n * (S * n + 1) / 2 * Lw; break;
                }
            }
            const int64_t w = static_cast<int64_t>(plan->S) * plan->n;
            plan->coeff_size = w * plan->H;
            const int L = plan->L, n = plan->n, H = plan->H;
            // prepare_soap, soap.cpp:507-534
            const double pi = 3.141592653589793238462643383279502884;
            const double eta = 1.0 / (2.0 * p.sigma * p.sigma);
            const double soap_scale = pi * std::sqrt(pi);
            plan->eta = eta;
            std::vector<double> pref(static_cast<size_t>(L * n), 1.0), expo(static_cast<size_t>(L * n), 0.0);
            std::vector<double> beta(static_cast<size_t>(L * n * n), 0.0);
            if (plan->radial_basis == 0) {
                double eta_power = 1.0;
                for (int l = 0; l < L; ++l) {
                    if (l > 0) eta_power *= eta;
                    for (int k = 0; k < n; ++k) {
                        const int idx = l * n + k;
                        const double alpha = p.alphas[idx];
                        const double denominator = alpha + eta;
                        pref[static_cast<size_t>(idx)] = eta_power * std::pow(denominator, -l - 1.5);
                        expo[static_cast<size_t>(idx)] = alpha * eta / denominator;
                    }
                }
                for (size_t i = 0; i < beta.size(); ++i) beta[i] = soap_scale * p.betas[i];
            } else {
                // polynomial: the per-neighbour radial functions G_lk come out
                // already projected (no fold), so the fold is the identity
                for (int l = 0; l < L; ++l) {
                    for (int k = 0; k < n; ++k) beta[static_cast<size_t>((l * n + k) * n + k)] = 1.0;
                }
                // quadrature-weighted basis values w_q r_q^2 g_k(r_q), [q * n + k] (soap.cpp:551-565)
                const int Q = o->grid_size;
                plan->grid_size = Q;
                std::vector<double> bw(static_cast<size_t>(Q) * n), grid(o->radial_grid, o->radial_grid + Q);
                for (int q = 0; q < Q; ++q) {
                    const double radial = o->radial_grid[q];
                    const double quadrature = o->radial_weights[q] * radial * radial;
                    for (int k = 0; k < n; ++k) {
                        bw[static_cast<size_t>(q) * n + k] = quadrature * o->radial_values[static_cast<size_t>(k) * Q + q];
                    }
                }
                upload(plan->d_poly_bw, bw);
                upload(plan->d_poly_grid, grid);
            }
            std::vector<double> ps_pref(static_cast<size_t>(L));
            for (int l = 0; l < L; ++l) ps_pref[static_cast<size_t>(l)] = pi * std::sqrt(8.0 / (2.0 * l + 1.0));
            // solid_harmonic_normalization (soap.cpp:26-38), sqrt(2) folded in for m > 0
            std::vector<double> hnorm(static_cast<size_t>(L * L), 0.0);
            const double sqrt2 = 1.414213562373095048801688724209698079;
            for (int l = 0; l < L; ++l) {
                for (int m = 0; m <= l; ++m) {
                    const double norm = std::sqrt((2.0 * l + 1.0) / (4.0 * pi)
                                                  * std::exp(std::lgamma(l - m + 1.0) - std::lgamma(l + m + 1.0)));
                    hnorm[static_cast<size_t>(l * L + m)] = m == 0 ? norm : sqrt2 * norm;
                }
            }
            // feature order of soap.cpp:997-1013 (labels core.py:321-329)
            std::vector<int32_t> fa, fb;
            fa.reserve(static_cast<size_t>(plan->features));
            fb.reserve(static_cast<size_t>(plan->features));
            for (int t1 = 0; t1 < plan->S; ++t1) {
                for (int t2 = t1; t2 < plan->S; ++t2) {
                    for (int l = 0; l < L; ++l) {
                        for (int n1 = 0; n1 < n; ++n1) {
                            for (int n2 = (t1 == t2 ? n1 : 0); n2 < n; ++n2) {
                                fa.push_back(((t1 * n + n1) * H + l * l) | (l << 24));
                                fb.push_back((t2 * n + n2) * H + l * l);
                            }
                        }
                    }
                }
            }
            // matrix-core paths unless MDX_HIP_SOAP_KERNEL=generic: the 4x4-block
            // kernel where the plan fits it, else the 16x16-tile kernel; =mfma
            // makes the 16x16-tile kernel mandatory, =quad the 4x4-block kernel
            const char* env = std::getenv("MDX_HIP_SOAP_KERNEL");
            const std::string choice = env != nullptr ? env : "auto";
            if (choice != "auto" && choice != "generic" && choice != "mfma" && choice != "quad" && choice != "block") {
                throw mdx::Error(MDX_INVALID_ARGUMENT, "MDX_HIP_SOAP_KERNEL must be auto, generic, mfma, quad or block");
            }
            const mdx::MfmaPlanHost mp = mdx::plan_mfma_tables(plan->Sc, n, p.l_max, beta, pref);
            mdx::MfmaDims md{};
            md.S = plan->S;
            md.Sc = plan->Sc;
            md.compression = plan->compression;
            md.radial = plan->radial_basis;
            md.grid = plan->grid_size;
            md.crow = mdx::mfma_coefficient_rows(plan->Sc, n, plan->compression);
            md.n = n;
            md.l_max = p.l_max;
            md.L = L;
            md.H = H;
            md.tiles = mp.tiles;
            md.mode = p.average;
            md.out_dtype = p.out_dtype;
            md.F = plan->features;
            md.hpad = mdx::mfma_padded_row(p.l_max);
            double max_expo = 0.0;
            for (double e : expo) max_expo = std::max(max_expo, e);
            md.clamp = max_expo * plan->cutoff * plan->cutoff > 700.0 ? 1 : 0;
            plan->hpad = md.hpad;
            plan->clamp = md.clamp;
            // the workgroup's LDS: 160 KiB on gfx950 (dynamic, no opt-in needed)
            const size_t lds_limit = mdx::device_workgroup_lds();
            const bool fits = mdx::mfma_template_tiles(mp.tiles) > 0 && mdx::mfma_lds_bytes(md) <= lds_limit;
            // only the matrix-core kernel implements weighting, compression and the polynomial basis
            const bool defaults = plan->compression == 0 && plan->radial_basis == 0 && plan->weighted == 0;
            plan->use_mfma = fits && (choice != "generic" || !defaults);
            if ((choice == "mfma" || !defaults) && !fits) {
                throw mdx::Error(MDX_INVALID_ARGUMENT, defaults
                    ? "SOAP shape is outside the matrix-core kernel's limits"
                    : "SOAP shape is outside the matrix-core kernel's limits, which weighting, compression and the "
                      "polynomial basis need");
            }
            plan->tiles = mp.tiles;
            const bool quad_range = -max_expo * plan->cutoff * plan->cutoff >= mdx::kQuadMinArgument;
            if (plan->use_mfma && defaults && quad_range && (choice == "auto" || choice == "quad")) {
                const mdx::QuadPlanHost qp = mdx::plan_quad_tables(n, p.l_max, md.hpad, beta, pref, expo);
                mdx::MfmaDims qd = md;
                qd.crow = mdx::quad_coefficient_rows(plan->Sc, n);
                if (qp.waves > 0 && mdx::quad_lds_bytes(qd) <= lds_limit) {
                    plan->quad_waves = qp.waves;
                    plan->quad_kg = qp.kg;
                    plan->quad_instr = qp.instr;
                    upload(plan->d_quad_lanes, qp.lanes);
                }
            }
            if (choice == "quad" && plan->quad_waves == 0) {
                throw mdx::Error(MDX_INVALID_ARGUMENT, "SOAP plan is outside the 4x4-block kernel's limits");
            }
            // register-coefficient kernel: GTO basis; atom-level rows with
            // compression off, mu2 or crossover (weighted or not) or mu1nu1
            // (unweighted), the same rows as float64 partial rows of an outer
            // average, or inner structure averages without compression
            // (weighted: large structures only); a compiled (l_max, radial
            // groups, species) shape.
            // It keeps its coefficients in registers, so the tile kernel's LDS
            // limit does not apply to it
            const int cm = plan->compression;
            const bool block_rows = (p.average == 0 || p.average == 2) &&
                                    (cm == 0 || cm == 1 || cm == 3 || (cm == 2 && plan->weighted == 0));
            const bool block_inner = p.average == 1 && cm == 0;
            const bool block_options = plan->radial_basis == 0 && (block_rows || block_inner);
            if (block_options && quad_range && (choice == "auto" || choice == "block")) {
                mdx::BlockPlanHost bp;
                // an outer average's rows are float64 partial rows
                const int row_dtype = p.average == 2 ? 8 : p.out_dtype;
                if (mdx::block_plan_tables(plan->S, n, p.l_max, row_dtype, cm, beta, pref, expo, bp)) {
                    plan->block_waves = bp.waves;
                    plan->block_kg = bp.kg;
                    plan->block_ncr = bp.ncr;
                    upload(plan->d_block_e1, bp.lane_e1);
                    upload(plan->d_block_beta, bp.lane_beta);
                    upload(plan->d_block_ps, bp.ps_offsets);
                }
            }
            plan->block_forced = choice == "block";
            if (choice == "block" && plan->block_waves == 0) {
                throw mdx::Error(MDX_INVALID_ARGUMENT, "SOAP plan is outside the register-coefficient kernel's shapes");
            }
            if (plan->use_mfma) {
                upload(plan->d_row_channel, mp.row_channel);
                upload(plan->d_col_harmonic, mp.col_harmonic);
                upload(plan->d_beta_lane, mp.beta_lane);
                upload(plan->d_fbase, mp.fbase);
                upload(plan->d_fstride, mp.fstride);
            }
            upload(plan->d_pref, pref);
            upload(plan->d_expo, expo);
            upload(plan->d_beta, beta);
            upload(plan->d_ps_pref, ps_pref);
            upload(plan->d_hnorm, hnorm);
            upload(plan->d_feat_a, fa);
            upload(plan->d_feat_b, fb);
            upload(plan->d_species_w, plan->species_weights);
        } catch (...) {
            delete plan;
            throw;
        }
        *out = plan;
        if (features != nullptr) *features = plan->features;
    });
}

void mdx_hip_soap_plan_destroy(mdx_soap_plan* plan) {
    if (plan == nullptr) return;
    int previous = -1;
    (void)hipGetDevice(&previous);
    (void)hipSetDevice(plan->device);
    delete plan;
    if (previous >= 0) (void)hipSetDevice(previous);
}

int64_t mdx_hip_soap_rows(const mdx_soap_plan* plan, const mdx_batch_view* batch) {
    if (plan == nullptr || batch == nullptr) return -1;
    return plan->average != 0 ? batch->structures : batch->atoms;
}

int mdx_hip_soap_compute(mdx_hip_ctx* ctx, const mdx_soap_plan* plan, const mdx_batch_view* batch, void* out_host,
                         int64_t out_rows, int64_t out_pitch_bytes, const volatile int32_t* cancel_flag,
                         mdx_timing* timing) {
    if (ctx == nullptr) return MDX_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(ctx->mutex);
    return guarded(ctx, [&] {
        if (plan == nullptr || batch == nullptr) throw mdx::Error(MDX_INVALID_ARGUMENT, "null plan or batch");
        if (plan->device != ctx->device) throw mdx::Error(MDX_INVALID_ARGUMENT, "plan belongs to another device");
        check_cancel(cancel_flag);
        DeviceScope scope(ctx->device);
        const int64_t rows = plan->average != 0 ? batch->structures : batch->atoms;
        const int64_t row_bytes = plan->features * plan->out_dtype;
        if (out_rows != rows) throw mdx::Error(MDX_INVALID_ARGUMENT, "output rows do not match the batch");
        if (out_pitch_bytes < row_bytes) throw mdx::Error(MDX_INVALID_ARGUMENT, "output pitch is too small");
        if (rows > 0 && row_bytes > 0 && out_host == nullptr) throw mdx::Error(MDX_INVALID_ARGUMENT, "null output");
        mdx::PreparedBatch& pb = ctx->scratch_batch;
        ctx->graph_kind = 0;
        pb.include_boundary = 1;
        mdx::prepare_batch(*batch, plan->species.data(), plan->S, plan->cutoff, pb);
        hipStream_t s = ctx->stream;
        MDX_HIP(hipEventRecord(ctx->events[5], s));
        mdx::upload_batch(s, *batch, pb);
        ctx->out_dev.reserve(std::max<size_t>(1, static_cast<size_t>(rows) * static_cast<size_t>(row_bytes)));
        if (plan->average == 0 && rows > 0 && row_bytes > 0 && is_pinned_host(out_host)) {
            // Atom-level rows into page-locked memory: the expansion runs in
            // about kOverlapSlices launches and each launch's rows go out on
            // the copy stream as soon as it finishes, so the PCIe transfer
            // (the longer part) overlaps the rest of the computation.
            constexpr int64_t kOverlapSlices = 8;
            const int64_t slice = std::max<int64_t>(4096, (rows + kOverlapSlices - 1) / kOverlapSlices);
            size_t next_event = 0;
            char* src = static_cast<char*>(ctx->out_dev.ptr);
            char* dst = static_cast<char*>(out_host);
            const mdx::SliceHook copy_rows = [&](int64_t first, int64_t count) {
                if (next_event == ctx->slice_events.size()) {
                    hipEvent_t ev = nullptr;
                    MDX_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
                    ctx->slice_events.push_back(ev);
                }
                hipEvent_t ev = ctx->slice_events[next_event++];
                MDX_HIP(hipEventRecord(ev, s));
                MDX_HIP(hipStreamWaitEvent(ctx->copy_stream, ev, 0));
                MDX_HIP(hipMemcpy2DAsync(dst + first * out_pitch_bytes, static_cast<size_t>(out_pitch_bytes),
                                         src + first * row_bytes, static_cast<size_t>(row_bytes),
                                         static_cast<size_t>(row_bytes), static_cast<size_t>(count),
                                         hipMemcpyDeviceToHost, ctx->copy_stream));
            };
            try {
                run_pipeline(ctx, *plan, pb, ctx->graph, ctx->partials, ctx->out_dev.ptr, row_bytes, cancel_flag,
                             timing, slice, &copy_rows);
            } catch (...) {
                (void)hipStreamSynchronize(ctx->copy_stream);
                throw;
            }
            ctx->graph_kind = 1;
            MDX_HIP(hipEventRecord(ctx->events[6], ctx->copy_stream));
            MDX_HIP(hipStreamSynchronize(ctx->copy_stream));
            MDX_HIP(hipStreamSynchronize(s));
            check_cancel(cancel_flag);
            // d2h_ms: the part of the transfer left after the last kernel
            fill_timing(ctx, timing, true);
            return;
        }
        run_pipeline(ctx, *plan, pb, ctx->graph, ctx->partials, ctx->out_dev.ptr, row_bytes, cancel_flag, timing);
        ctx->graph_kind = 1;
        MDX_HIP(hipStreamSynchronize(s));
        check_cancel(cancel_flag);
        const auto t0 = std::chrono::steady_clock::now();
        download_result(ctx, ctx->out_dev.ptr, rows, row_bytes, out_host, out_pitch_bytes);
        const auto t1 = std::chrono::steady_clock::now();
        MDX_HIP(hipEventRecord(ctx->events[6], s));
        MDX_HIP(hipStreamSynchronize(s));
        fill_timing(ctx, timing, true);
        if (timing != nullptr) timing->d2h_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    });
}

int mdx_hip_batch_upload(mdx_hip_ctx* ctx, const mdx_soap_plan* plan, const mdx_batch_view* batch,
                         mdx_device_batch** out) {
    if (ctx == nullptr || out == nullptr) return MDX_INVALID_ARGUMENT;
    *out = nullptr;
    std::lock_guard<std::mutex> lock(ctx->mutex);
    return guarded(ctx, [&] {
        if (plan == nullptr || batch == nullptr) throw mdx::Error(MDX_INVALID_ARGUMENT, "null plan or batch");
        if (plan->device != ctx->device) throw mdx::Error(MDX_INVALID_ARGUMENT, "plan belongs to another device");
        DeviceScope scope(ctx->device);
        auto db = new mdx_device_batch();
        try {
            db->device = ctx->device;
            db->pb.include_boundary = 1;
            mdx::prepare_batch(*batch, plan->species.data(), plan->S, plan->cutoff, db->pb);
            mdx::upload_batch(ctx->stream, *batch, db->pb);
            // the host copy from which pipelined frames prepare their second set
            const size_t atoms = static_cast<size_t>(batch->atoms), structures = static_cast<size_t>(batch->structures);
            db->host_numbers.assign(batch->numbers, batch->numbers + atoms);
            db->host_positions.assign(batch->positions, batch->positions + 3 * atoms);
            db->host_cells.assign(batch->cells, batch->cells + 9 * structures);
            db->host_pbc.assign(batch->pbc, batch->pbc + 3 * structures);
            db->host_offsets.assign(batch->offsets, batch->offsets + structures + 1);
        } catch (...) {
            delete db;
            throw;
        }
        *out = db;
    });
}

namespace {

// The stream on which a pipelined frame of buffer set k builds its graph:
// one per set, so that the next frame's graph starts while this one's search
// still runs (the second is the context's copy stream, which the host-batch
// path uses only inside its own synchronous calls).
hipStream_t frame_stream(const mdx_hip_ctx* ctx, int k) { return k == 0 ? ctx->graph_stream : ctx->copy_stream; }

// The statistics of the batch's last pipelined frame, read once its search
// has finished.  A centre that overflowed its slot (the queued expansion then
// read clamped rows) has the frame built again on the compact layout from the
// positions still in its set and expanded again into its output, on the main
// stream behind the expansion that was wrong and before any later one.
void settle(mdx_hip_ctx* ctx, mdx_device_batch* batch) {
    const int j = batch->pending;
    if (j < 0) return;
    batch->pending = -1;
    mdx::PreparedBatch& pb = j == 0 ? batch->pb : *batch->pb2;
    mdx::DeviceGraph& graph = j == 0 ? batch->graph : batch->graph2;
    mdx::DeviceBuffer& partials = j == 0 ? batch->partials : batch->partials2;
    const volatile int32_t* cancel = batch->pending_cancel;
    if (mdx::complete_graph(pb, graph, cancel)) return;
    hipStream_t s = ctx->stream;
    MDX_HIP(hipStreamSynchronize(s)); // the first expansion's buffers are replaced
    MDX_HIP(hipStreamSynchronize(frame_stream(ctx, j)));
    mdx::build_graph(s, pb, graph, cancel, true, false, true);
    check_cancel(cancel);
    mdx::run_soap(s, *batch->pending_plan, pb, graph, batch->pending_out, batch->pending_pitch, partials, cancel,
                  nullptr, nullptr);
    MDX_HIP(hipEventRecord(batch->done[j], s));
}

// Settle the batch's pipelined frames and wait for them (their expansions
// read its sets), so that a synchronous call may reuse set 0.
void quiesce(mdx_hip_ctx* ctx, mdx_device_batch* batch) {
    settle(ctx, batch);
    for (int k = 0; k < 2; ++k) {
        if (batch->queued[k]) {
            MDX_HIP(hipEventSynchronize(batch->done[k]));
            batch->queued[k] = false;
        }
    }
}

} // namespace

int mdx_hip_batch_set_positions(mdx_hip_ctx* ctx, mdx_device_batch* batch, const double* positions) {
    if (ctx == nullptr) return MDX_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(ctx->mutex);
    return guarded(ctx, [&] {
        if (batch == nullptr) throw mdx::Error(MDX_INVALID_ARGUMENT, "null batch");
        if (batch->device != ctx->device) throw mdx::Error(MDX_INVALID_ARGUMENT, "batch belongs to another device");
        const size_t values = static_cast<size_t>(batch->pb.atoms) * 3;
        if (values == 0) return;
        if (positions == nullptr) throw mdx::Error(MDX_INVALID_ARGUMENT, "null positions");
        DeviceScope scope(ctx->device);
        quiesce(ctx, batch);
        if (is_device_memory(positions)) {
            // checked for finiteness by the next run's frame kernels
            MDX_HIP(hipMemcpyAsync(batch->pb.d_positions.ptr, positions, values * sizeof(double),
                                   hipMemcpyDeviceToDevice, ctx->stream));
            return;
        }
        for (size_t i = 0; i < values; ++i) {
            if (!std::isfinite(positions[i])) throw mdx::Error(MDX_INVALID_ARGUMENT, "positions must be finite");
        }
        MDX_HIP(hipMemcpyAsync(batch->pb.d_positions.ptr, positions, values * sizeof(double), hipMemcpyHostToDevice,
                               ctx->stream));
        MDX_HIP(hipStreamSynchronize(ctx->stream));
    });
}

void mdx_hip_batch_destroy(mdx_device_batch* batch) {
    if (batch == nullptr) return;
    int previous = -1;
    (void)hipGetDevice(&previous);
    (void)hipSetDevice(batch->device);
    delete batch;
    if (previous >= 0) (void)hipSetDevice(previous);
}

namespace {

// Arguments of a device-batch run, checked as mdx_hip_soap_run documents.
void check_device_run(const mdx_hip_ctx* ctx, const mdx_soap_plan* plan, const mdx_device_batch* batch,
                      const void* out_device, int64_t out_pitch_bytes) {
    if (plan == nullptr || batch == nullptr) throw mdx::Error(MDX_INVALID_ARGUMENT, "null plan or batch");
    if (plan->device != ctx->device || batch->device != ctx->device) {
        throw mdx::Error(MDX_INVALID_ARGUMENT, "plan or batch belongs to another device");
    }
    if (batch->pb.n_species != plan->S || batch->pb.cutoff != plan->cutoff) {
        throw mdx::Error(MDX_INVALID_ARGUMENT, "device batch was prepared for another plan");
    }
    const int64_t rows = plan->average != 0 ? batch->pb.structures : batch->pb.atoms;
    const int64_t row_bytes = plan->features * plan->out_dtype;
    if (out_pitch_bytes < row_bytes) throw mdx::Error(MDX_INVALID_ARGUMENT, "output pitch is too small");
    if (rows > 0 && row_bytes > 0 && out_device == nullptr) throw mdx::Error(MDX_INVALID_ARGUMENT, "null output");
}

} // namespace

int mdx_hip_soap_run(mdx_hip_ctx* ctx, const mdx_soap_plan* plan, mdx_device_batch* batch, void* out_device,
                     int64_t out_pitch_bytes, const volatile int32_t* cancel_flag, mdx_timing* timing) {
    if (ctx == nullptr) return MDX_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(ctx->mutex);
    return guarded(ctx, [&] {
        check_device_run(ctx, plan, batch, out_device, out_pitch_bytes);
        check_cancel(cancel_flag);
        DeviceScope scope(ctx->device);
        quiesce(ctx, batch);
        run_pipeline(ctx, *plan, batch->pb, batch->graph, batch->partials, out_device, out_pitch_bytes, cancel_flag,
                     timing);
        ctx->finished.wait(ctx->stream);
        fill_timing(ctx, timing, false);
    });
}

int mdx_hip_soap_run_noalloc(mdx_hip_ctx* ctx, const mdx_soap_plan* plan, mdx_device_batch* batch,
                             void* out_device, int64_t out_pitch_bytes, const volatile int32_t* cancel_flag,
                             mdx_timing* timing) {
    if (ctx == nullptr) return MDX_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(ctx->mutex);
    return guarded(ctx, [&] {
        check_device_run(ctx, plan, batch, out_device, out_pitch_bytes);
        check_cancel(cancel_flag);
        DeviceScope scope(ctx->device);
        quiesce(ctx, batch);
        // every piece is carved afresh from the start of the array; the
        // graph's counters are cleared on the stream before each build
        ctx->arena.reset();
        ctx->static_graph.for_each_buffer([](mdx::DeviceBuffer& b) { b.release(); });
        ctx->static_partials.release();
        run_pipeline(ctx, *plan, batch->pb, ctx->static_graph, ctx->static_partials, out_device, out_pitch_bytes,
                     cancel_flag, timing);
        ctx->finished.wait(ctx->stream);
        fill_timing(ctx, timing, false);
    });
}

int mdx_hip_soap_run_frame(mdx_hip_ctx* ctx, const mdx_soap_plan* plan, mdx_device_batch* batch,
                           const double* positions, void* out_device, int64_t out_pitch_bytes,
                           const volatile int32_t* cancel_flag) {
    if (ctx == nullptr) return MDX_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(ctx->mutex);
    return guarded(ctx, [&] {
        check_device_run(ctx, plan, batch, out_device, out_pitch_bytes);
        check_cancel(cancel_flag);
        const size_t values = static_cast<size_t>(batch->pb.atoms) * 3;
        if (values > 0 && positions == nullptr) throw mdx::Error(MDX_INVALID_ARGUMENT, "null positions");
        DeviceScope scope(ctx->device);
        const int k = batch->next_set;
        if (k == 1 && batch->pb2 == nullptr) {
            // the second set: the batch prepared again from its host copy
            auto pb2 = std::make_unique<mdx::PreparedBatch>();
            const mdx_batch_view view{batch->host_numbers.data(), batch->host_positions.data(),
                                      batch->host_cells.data(), batch->host_pbc.data(), batch->host_offsets.data(),
                                      static_cast<int64_t>(batch->host_offsets.size()) - 1,
                                      static_cast<int64_t>(batch->host_numbers.size())};
            pb2->include_boundary = 1;
            mdx::prepare_batch(view, plan->species.data(), plan->S, plan->cutoff, *pb2);
            mdx::upload_batch(frame_stream(ctx, 1), view, *pb2);
            batch->pb2 = std::move(pb2);
        }
        for (int e = 0; e < 2; ++e) {
            if (batch->ready[e] == nullptr) MDX_HIP(hipEventCreateWithFlags(&batch->ready[e], hipEventDisableTiming));
            if (batch->done[e] == nullptr) MDX_HIP(hipEventCreateWithFlags(&batch->done[e], hipEventDisableTiming));
        }
        mdx::PreparedBatch& pb = k == 0 ? batch->pb : *batch->pb2;
        mdx::DeviceGraph& graph = k == 0 ? batch->graph : batch->graph2;
        mdx::DeviceBuffer& partials = k == 0 ? batch->partials : batch->partials2;
        // the set's buffers are rebuilt (and may be reallocated) only after
        // the expansion that last read them has finished; that frame was
        // settled by the call after it
        if (batch->queued[k]) {
            MDX_HIP(hipEventSynchronize(batch->done[k]));
            batch->queued[k] = false;
        }
        hipStream_t gs = frame_stream(ctx, k), s = ctx->stream;
        if (values > 0) {
            if (is_device_memory(positions)) {
                // checked for finiteness by the frame kernels below
                MDX_HIP(hipMemcpyAsync(pb.d_positions.ptr, positions, values * sizeof(double),
                                       hipMemcpyDeviceToDevice, gs));
            } else {
                for (size_t i = 0; i < values; ++i) {
                    if (!std::isfinite(positions[i])) {
                        throw mdx::Error(MDX_INVALID_ARGUMENT, "positions must be finite");
                    }
                }
                MDX_HIP(hipMemcpyAsync(pb.d_positions.ptr, positions, values * sizeof(double),
                                       hipMemcpyHostToDevice, gs));
            }
        }
        // this frame's graph on its set's stream, beside the previous frame's
        // search and expansion (the call returns from the frame read-back
        // with the search queued); its expansion on the main stream behind
        // the graph and the previous frame, which is settled first
        mdx::build_graph(gs, pb, graph, cancel_flag, true, true);
        MDX_HIP(hipEventRecord(batch->ready[k], gs));
        settle(ctx, batch);
        MDX_HIP(hipStreamWaitEvent(s, batch->ready[k], 0));
        check_cancel(cancel_flag);
        // (a weighted plan's per-row weight pass goes behind the graph on gs)
        mdx::run_soap(s, *plan, pb, graph, out_device, out_pitch_bytes, partials, cancel_flag, nullptr, nullptr, 0,
                      nullptr, gs, batch->ready[k]);
        MDX_HIP(hipEventRecord(batch->done[k], s));
        batch->queued[k] = true;
        batch->pending = k;
        batch->pending_plan = plan;
        batch->pending_out = out_device;
        batch->pending_pitch = out_pitch_bytes;
        batch->pending_cancel = cancel_flag;
        batch->next_set = k ^ 1;
    });
}

int mdx_hip_batch_wait(mdx_hip_ctx* ctx, mdx_device_batch* batch) {
    if (ctx == nullptr) return MDX_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(ctx->mutex);
    return guarded(ctx, [&] {
        if (batch == nullptr) throw mdx::Error(MDX_INVALID_ARGUMENT, "null batch");
        if (batch->device != ctx->device) throw mdx::Error(MDX_INVALID_ARGUMENT, "batch belongs to another device");
        DeviceScope scope(ctx->device);
        quiesce(ctx, batch);
    });
}

int mdx_hip_neighbors_build(mdx_hip_ctx* ctx, const mdx_batch_view* batch, double cutoff, int32_t include_boundary,
                            int64_t* pairs) {
    if (ctx == nullptr) return MDX_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(ctx->mutex);
    return guarded(ctx, [&] {
        if (batch == nullptr) throw mdx::Error(MDX_INVALID_ARGUMENT, "null batch");
        DeviceScope scope(ctx->device);
        mdx::PreparedBatch& pb = ctx->scratch_batch;
        ctx->graph_kind = 0;
        pb.include_boundary = include_boundary != 0 ? 1 : 0;
        mdx::prepare_batch(*batch, nullptr, 1, cutoff, pb);
        mdx::upload_batch(ctx->stream, *batch, pb);
        const int64_t n = mdx::build_graph(ctx->stream, pb, ctx->graph, nullptr);
        MDX_HIP(hipStreamSynchronize(ctx->stream));
        ctx->graph_kind = 2;
        if (pairs != nullptr) *pairs = n;
    });
}

int mdx_hip_neighbors_fetch(mdx_hip_ctx* ctx, int64_t* offsets, int32_t* neighbors, int32_t* shifts,
                            double* displacements, double* distance2) {
    if (ctx == nullptr) return MDX_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(ctx->mutex);
    return guarded(ctx, [&] {
        DeviceScope scope(ctx->device);
        const mdx::PreparedBatch& pb = ctx->scratch_batch;
        mdx::DeviceGraph& g = ctx->graph;
        if (ctx->graph_kind != 2) throw mdx::Error(MDX_INVALID_ARGUMENT, "no neighbour graph has been built");
        hipStream_t s = ctx->stream;
        const int64_t atoms = pb.atoms, pairs = g.pairs;
        if (offsets != nullptr) {
            MDX_HIP(hipMemcpyAsync(offsets, g.pair_start.ptr, static_cast<size_t>(atoms + 1) * sizeof(int64_t),
                                   hipMemcpyDeviceToHost, s));
        }
        if (pairs > 0) {
            mdx::DeviceBuffer& tmp = ctx->out_dev;
            const size_t p = static_cast<size_t>(pairs);
            tmp.reserve(p * (4 + 12 + 24 + 8));
            char* base = static_cast<char*>(tmp.ptr);
            double* d_disp = reinterpret_cast<double*>(base);
            double* d_d2 = d_disp + 3 * p;
            int32_t* d_atoms = reinterpret_cast<int32_t*>(d_d2 + p);
            int32_t* d_shifts = d_atoms + p;
            const unsigned grid = static_cast<unsigned>(std::min<int64_t>((pairs + 255) / 256, 1 << 20));
            hipLaunchKernelGGL(k_export_pairs, dim3(grid), dim3(256), 0, s, g.pair_start.as<int64_t>(), atoms, pairs,
                               g.pair_bin.as<uint32_t>(), pb.d_positions.as<double>(), g.bin_x.as<double>(),
                               g.bin_y.as<double>(), g.bin_z.as<double>(), g.bin_atom.as<int32_t>(),
                               g.bin_image.as<int32_t>(), pb.d_images.as<mdx::ImageDesc>(), d_atoms, d_shifts, d_disp,
                               d_d2);
            MDX_HIP(hipGetLastError());
            if (neighbors != nullptr) MDX_HIP(hipMemcpyAsync(neighbors, d_atoms, p * 4, hipMemcpyDeviceToHost, s));
            if (shifts != nullptr) MDX_HIP(hipMemcpyAsync(shifts, d_shifts, p * 12, hipMemcpyDeviceToHost, s));
            if (displacements != nullptr) {
                MDX_HIP(hipMemcpyAsync(displacements, d_disp, p * 24, hipMemcpyDeviceToHost, s));
            }
            if (distance2 != nullptr) MDX_HIP(hipMemcpyAsync(distance2, d_d2, p * 8, hipMemcpyDeviceToHost, s));
        }
        MDX_HIP(hipStreamSynchronize(s));
    });
}

int mdx_hip_neighbor_list(mdx_hip_ctx* ctx, const mdx_batch_view* batch, double cutoff, int32_t full_neighbor_list,
                          int32_t self_pairs, const volatile int32_t* cancel_flag, int64_t* pairs) {
    if (ctx == nullptr) return MDX_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(ctx->mutex);
    return guarded(ctx, [&] {
        if (batch == nullptr) throw mdx::Error(MDX_INVALID_ARGUMENT, "null batch");
        check_cancel(cancel_flag);
        DeviceScope scope(ctx->device);
        mdx::PreparedBatch& pb = ctx->scratch_batch;
        ctx->graph_kind = 0;
        pb.include_boundary = 1; // build_neighbor_graph's default (cpp/include/mdescriptor/neighbor.hpp:50-57)
        mdx::prepare_batch(*batch, nullptr, 1, cutoff, pb);
        mdx::upload_batch(ctx->stream, *batch, pb);
        ctx->list_filled = false;
        MDX_HIP(hipEventRecord(ctx->list_events[0], ctx->stream));
        // one search pass into per-centre slots (the compact two-pass layout
        // when a centre overflows its slot); the list kernels read each
        // centre's rows in the reference's order either way
        mdx::build_graph(ctx->stream, pb, ctx->graph, cancel_flag, true);
        MDX_HIP(hipEventRecord(ctx->list_events[1], ctx->stream));
        check_cancel(cancel_flag);
        const int64_t rows = mdx::count_neighbor_list(ctx->stream, pb, ctx->graph, full_neighbor_list != 0 ? 1 : 0,
                                                      self_pairs != 0 ? 1 : 0, ctx->list, ctx->list_events[2]);
        ctx->graph_kind = 3;
        if (pairs != nullptr) *pairs = rows;
    });
}

int mdx_hip_neighbor_list_fetch(mdx_hip_ctx* ctx, double* table, double* values, int64_t* samples,
                                int64_t* offsets) {
    if (ctx == nullptr) return MDX_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(ctx->mutex);
    return guarded(ctx, [&] {
        if (ctx->graph_kind != 3) throw mdx::Error(MDX_INVALID_ARGUMENT, "no neighbour list has been computed");
        DeviceScope scope(ctx->device);
        const mdx::PreparedBatch& pb = ctx->scratch_batch;
        const int64_t rows = ctx->list.rows;
        hipStream_t s = ctx->stream;
        // device destinations with the alignment of the fill kernel's 8-byte
        // stores are written in place; host ones (and misaligned device
        // ones) through a device staging area, one region per output
        struct Target {
            void* user;
            int64_t count;     // records
            int64_t width;     // bytes per record
            uintptr_t align;   // alignment of the kernel's stores
            void* device = nullptr;
            bool on_device = false;
            size_t bytes() const { return static_cast<size_t>(count) * static_cast<size_t>(width); }
        };
        Target t[4] = {{table, rows, 72, 8}, {values, rows, 32, 8}, {samples, rows, 48, 8},
                       {offsets, pb.structures + 1, static_cast<int64_t>(sizeof(int64_t)), 8}};
        size_t staged = 0;
        for (Target& x : t) {
            if (x.user == nullptr || x.bytes() == 0) continue;
            x.on_device = is_device_memory(x.user);
            if (x.on_device && reinterpret_cast<uintptr_t>(x.user) % x.align == 0) {
                x.device = x.user;
            } else {
                x.device = reinterpret_cast<void*>(staged); // offset, rebased below
                staged += (x.bytes() + 255) & ~size_t(255);
            }
        }
        if (staged > 0) {
            ctx->out_dev.reserve(staged);
            for (Target& x : t) {
                if (x.user != nullptr && x.bytes() != 0 && x.device != x.user) {
                    x.device = static_cast<char*>(ctx->out_dev.ptr) + reinterpret_cast<size_t>(x.device);
                }
            }
        }
        MDX_HIP(hipEventRecord(ctx->list_events[3], s));
        mdx::fill_neighbor_list(s, pb, ctx->graph, ctx->list, static_cast<double*>(t[0].device),
                                static_cast<double*>(t[1].device), static_cast<int64_t*>(t[2].device),
                                static_cast<int64_t*>(t[3].device));
        MDX_HIP(hipEventRecord(ctx->list_events[4], s));
        ctx->list_filled = true;
        for (Target& x : t) {
            if (x.device == nullptr || x.device == x.user) continue;
            if (x.on_device) {
                MDX_HIP(hipMemcpyAsync(x.user, x.device, x.bytes(), hipMemcpyDeviceToDevice, s));
            } else {
                download_result(ctx, x.device, x.count, x.width, x.user, x.width);
            }
        }
        MDX_HIP(hipStreamSynchronize(s));
    });
}

int mdx_hip_neighbor_list_timing(mdx_hip_ctx* ctx, mdx_list_timing* timing) {
    if (ctx == nullptr || timing == nullptr) return MDX_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(ctx->mutex);
    return guarded(ctx, [&] {
        if (ctx->graph_kind != 3) throw mdx::Error(MDX_INVALID_ARGUMENT, "no neighbour list has been computed");
        DeviceScope scope(ctx->device);
        MDX_HIP(hipStreamSynchronize(ctx->stream));
        *timing = mdx_list_timing{};
        timing->graph_ms = elapsed(ctx->list_events[0], ctx->list_events[1]);
        timing->count_ms = elapsed(ctx->list_events[1], ctx->list_events[2]);
        timing->fill_ms = ctx->list_filled ? elapsed(ctx->list_events[3], ctx->list_events[4]) : 0.0;
        timing->graph_pairs = ctx->graph.pairs;
        timing->pairs = ctx->list.rows;
        timing->binned = ctx->graph.binned;
    });
}

} // extern "C"
