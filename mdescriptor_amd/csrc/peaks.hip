// Peak-rate probes of the device the roofline is quoted against: FP64 FMA
// on the vector ALU, FP64 16x16x4 matrix-core MFMA, and an HBM copy.  A
// diagnostic library of its own (libmdx_peaks.so), loaded by bench.py
// --peaks; the SOAP library does not use it.
//
// Each probe is timed with HIP events around `repeats` launches on its own
// stream and reports seconds per launch and work per launch (flops or
// bytes moved, read plus write).
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int kBlock = 256;
constexpr int kChains = 8;   // independent FMA chains per lane
constexpr int kAcc = 4;      // independent MFMA accumulators per wavefront

__global__ __launch_bounds__(kBlock) void k_fma_f64(double* out, int iterations, double b, double c) {
    double a[kChains];
#pragma unroll
    for (int k = 0; k < kChains; ++k) a[k] = static_cast<double>(threadIdx.x + k);
    for (int i = 0; i < iterations; ++i) {
#pragma unroll
        for (int k = 0; k < kChains; ++k) a[k] = fma(a[k], b, c);
    }
    double sum = 0.0;
#pragma unroll
    for (int k = 0; k < kChains; ++k) sum += a[k];
    // keep the chains live; b and c keep the values finite (|b| < 1)
    if (sum == 12345.678) out[blockIdx.x * kBlock + threadIdx.x] = sum;
}

typedef double d4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kBlock) void k_mfma_f64(double* out, int iterations, double b) {
    d4 acc[kAcc];
#pragma unroll
    for (int k = 0; k < kAcc; ++k) acc[k] = d4{0.0, 0.0, 0.0, 0.0};
    const double a = static_cast<double>(threadIdx.x) * 1e-3;
    for (int i = 0; i < iterations; ++i) {
#pragma unroll
        for (int k = 0; k < kAcc; ++k) acc[k] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, acc[k], 0, 0, 0);
    }
    double sum = 0.0;
#pragma unroll
    for (int k = 0; k < kAcc; ++k) sum += acc[k][0] + acc[k][1] + acc[k][2] + acc[k][3];
    if (sum == 12345.678) out[blockIdx.x * kBlock + threadIdx.x] = sum;
}

__global__ __launch_bounds__(kBlock) void k_copy(const double4* src, double4* dst, int64_t n) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(kBlock) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kBlock) {
        dst[i] = src[i];
    }
}

// Streaming forms: each thread moves kUnroll 16-byte vectors per iteration,
// all loads issued before the stores, with non-temporal hints (the data is
// touched once: no reason to keep it in the caches).  n16 counts 16-byte
// vectors and is a multiple of kUnroll * kBlock * gridDim.x (the host sizes
// the buffer so), so no iteration needs a bounds check per vector.
constexpr int kUnroll = 4;
typedef unsigned int u4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kBlock) void k_copy_stream(const u4* src, u4* dst, int64_t n16) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock * kUnroll;
    for (int64_t base = (blockIdx.x * static_cast<int64_t>(kBlock)) * kUnroll + threadIdx.x; base < n16;
         base += stride) {
        u4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) v[u] = __builtin_nontemporal_load(&src[base + u * kBlock]);
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) __builtin_nontemporal_store(v[u], &dst[base + u * kBlock]);
    }
}

__global__ __launch_bounds__(kBlock) void k_read_stream(const u4* src, int64_t n16, unsigned* out) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock * kUnroll;
    unsigned acc = 0;
    for (int64_t base = (blockIdx.x * static_cast<int64_t>(kBlock)) * kUnroll + threadIdx.x; base < n16;
         base += stride) {
        u4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) v[u] = __builtin_nontemporal_load(&src[base + u * kBlock]);
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    // keep the loads live (the buffer is zero-filled: never taken)
    if (acc == 0x9e3779b9u) out[blockIdx.x * kBlock + threadIdx.x] = acc;
}

__global__ __launch_bounds__(kBlock) void k_write_stream(u4* dst, int64_t n16) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock * kUnroll;
    const u4 v = {threadIdx.x, blockIdx.x, 0u, 1u};
    for (int64_t base = (blockIdx.x * static_cast<int64_t>(kBlock)) * kUnroll + threadIdx.x; base < n16;
         base += stride) {
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) __builtin_nontemporal_store(v, &dst[base + u * kBlock]);
    }
}

int device_cus() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    return cus;
}

} // namespace

extern "C" {

// which: 0 FP64 FMA (vector ALU), 1 FP64 MFMA 16x16x4, 2 HBM copy of `size`
// bytes (32-byte elements, grid-stride), 3 the same copy streamed (16-byte
// vectors, four per thread in flight, non-temporal), 4 a streamed read of
// `size` bytes, 5 a streamed write of `size` bytes.  Returns 0 on success,
// else the HIP error code.  *seconds receives the time per launch, *work the
// flops (0, 1) or bytes read + written (2-5) per launch.
int mdx_peak_run(int which, int64_t size, int repeats, double* seconds, double* work) {
    const int cus = device_cus();
    if (cus <= 0 || repeats <= 0 || seconds == nullptr || work == nullptr) return 1;
    hipStream_t stream = nullptr;
    hipEvent_t start = nullptr, stop = nullptr;
    void* a = nullptr;
    void* b = nullptr;
    hipError_t rc = hipStreamCreateWithFlags(&stream, hipStreamNonBlocking);
    if (rc == hipSuccess) rc = hipEventCreate(&start);
    if (rc == hipSuccess) rc = hipEventCreate(&stop);
    // enough workgroups for 8 wavefronts per SIMD on every CU
    const unsigned grid = static_cast<unsigned>(cus) * 8;
    const int iterations = 4096;
    const bool memory = which >= 2;
    // the streamed probes move whole rounds of the grid: size rounded down to
    // a multiple of grid * 4 (workgroups) * kBlock * kUnroll * 16 bytes
    const size_t round = static_cast<size_t>(grid) * 4 * kBlock * kUnroll * 16;
    const size_t bytes = !memory ? grid * kBlock * sizeof(double)
                         : which == 2 ? static_cast<size_t>(size)
                                      : static_cast<size_t>(size) / round * round;
    if (memory && bytes == 0) return 1;
    if (rc == hipSuccess) rc = hipMalloc(&a, bytes);
    if (rc == hipSuccess && (which == 2 || which == 3 || which == 4)) rc = hipMalloc(&b, which == 4 ? round : bytes);
    if (rc == hipSuccess && memory) rc = hipMemsetAsync(a, 0, bytes, stream);
    auto launch = [&]() {
        if (which == 0) {
            hipLaunchKernelGGL(k_fma_f64, dim3(grid), dim3(kBlock), 0, stream, static_cast<double*>(a), iterations,
                               0.999999, 1e-7);
        } else if (which == 1) {
            hipLaunchKernelGGL(k_mfma_f64, dim3(grid), dim3(kBlock), 0, stream, static_cast<double*>(a), iterations,
                               1e-6);
        } else if (which == 2) {
            const int64_t n = static_cast<int64_t>(bytes / sizeof(double4));
            hipLaunchKernelGGL(k_copy, dim3(grid * 4), dim3(kBlock), 0, stream, static_cast<const double4*>(a),
                               static_cast<double4*>(b), n);
        } else {
            const int64_t n16 = static_cast<int64_t>(bytes / 16);
            if (which == 3) {
                hipLaunchKernelGGL(k_copy_stream, dim3(grid * 4), dim3(kBlock), 0, stream,
                                   static_cast<const u4*>(a), static_cast<u4*>(b), n16);
            } else if (which == 4) {
                hipLaunchKernelGGL(k_read_stream, dim3(grid * 4), dim3(kBlock), 0, stream,
                                   static_cast<const u4*>(a), n16, static_cast<unsigned*>(b));
            } else {
                hipLaunchKernelGGL(k_write_stream, dim3(grid * 4), dim3(kBlock), 0, stream, static_cast<u4*>(a), n16);
            }
        }
    };
    if (rc == hipSuccess) {
        launch(); // warm-up
        rc = hipEventRecord(start, stream);
    }
    if (rc == hipSuccess) {
        for (int r = 0; r < repeats; ++r) launch();
        rc = hipGetLastError();
    }
    if (rc == hipSuccess) rc = hipEventRecord(stop, stream);
    if (rc == hipSuccess) rc = hipEventSynchronize(stop);
    float ms = 0.0f;
    if (rc == hipSuccess) rc = hipEventElapsedTime(&ms, start, stop);
    if (rc == hipSuccess) {
        *seconds = static_cast<double>(ms) * 1e-3 / repeats;
        const double threads = static_cast<double>(grid) * kBlock;
        if (which == 0) {
            *work = 2.0 * kChains * iterations * threads;
        } else if (which == 1) {
            *work = 2.0 * 16 * 16 * 4 * kAcc * iterations * (threads / 64.0);
        } else if (which == 2) {
            *work = 2.0 * static_cast<double>(bytes / sizeof(double4) * sizeof(double4));
        } else {
            *work = (which == 3 ? 2.0 : 1.0) * static_cast<double>(bytes);
        }
    }
    if (a != nullptr) (void)hipFree(a);
    if (b != nullptr) (void)hipFree(b);
    if (start != nullptr) (void)hipEventDestroy(start);
    if (stop != nullptr) (void)hipEventDestroy(stop);
    if (stream != nullptr) (void)hipStreamDestroy(stream);
    return rc == hipSuccess ? 0 : static_cast<int>(rc);
}

} // extern "C"
