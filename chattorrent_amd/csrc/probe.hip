// Bandwidth probes for the benchmark (libccprobe.so, C ABI): the practical
// HBM ceilings the decode pass is compared with, measured on the same GPU in
// the same process. Not part of the decode library.
//
//   ccp_read_gbps: a read-only stream (16-byte vector loads over a buffer far
//     larger than the 256 MiB Infinity Cache, every wave on its own forward
//     run, the loaded words folded so the loads are kept) — the ceiling of a
//     pass that almost only reads;
//   ccp_copy_gbps: a device-to-device copy (bytes read + bytes written).
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int kThreads = 256;

// Each workgroup streams one contiguous span; its lanes read consecutive
// 16-byte words, four loads in flight per lane.
__global__ __launch_bounds__(kThreads) void k_read(const u32x4* __restrict__ p, size_t n16, uint32_t* sink) {
    const size_t span = (n16 + gridDim.x - 1) / gridDim.x;
    const size_t a = (size_t)blockIdx.x * span, b = a + span < n16 ? a + span : n16;
    uint32_t acc = 0;
    size_t i = a + threadIdx.x;
    for (; i + 3 * kThreads < b; i += 4 * kThreads) {
        const u32x4 v0 = p[i], v1 = p[i + kThreads], v2 = p[i + 2 * kThreads], v3 = p[i + 3 * kThreads];
        acc ^= v0[0] ^ v1[1] ^ v2[2] ^ v3[3];
    }
    for (; i < b; i += kThreads) acc ^= p[i][0];
    if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;   // practically never; keeps the loads
}

__global__ __launch_bounds__(kThreads) void k_copy(const u32x4* __restrict__ s, u32x4* __restrict__ d, size_t n16) {
    for (size_t i = blockIdx.x * (size_t)kThreads + threadIdx.x; i < n16; i += (size_t)gridDim.x * kThreads) d[i] = s[i];
}

int run(int device, size_t bytes, int iters, bool copy, double* gbps) {
    if (!gbps || bytes < (1u << 20) || iters < 1) return 1;
    if (hipSetDevice(device) != hipSuccess) return 2;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return 2;
    const size_t n16 = bytes / 16;
    u32x4 *a = nullptr, *b = nullptr;
    uint32_t* sink = nullptr;
    hipStream_t st = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = 3;
    const int grid = prop.multiProcessorCount * 16;
    float ms = 0.f;
    if (hipMalloc(&a, n16 * 16) != hipSuccess) goto done;
    if (copy && hipMalloc(&b, n16 * 16) != hipSuccess) goto done;
    if (hipMalloc(&sink, (size_t)grid * 4) != hipSuccess) goto done;
    if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess) goto done;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) goto done;
    if (hipMemsetAsync(a, 0x5a, n16 * 16, st) != hipSuccess) goto done;
    for (int r = -1; r < iters; r++) {   // one untimed pass first
        if (r == 0 && hipEventRecord(e0, st) != hipSuccess) goto done;
        if (copy) hipLaunchKernelGGL(k_copy, dim3(grid), dim3(kThreads), 0, st, a, b, n16);
        else hipLaunchKernelGGL(k_read, dim3(grid), dim3(kThreads), 0, st, a, n16, sink);
    }
    if (hipEventRecord(e1, st) != hipSuccess || hipEventSynchronize(e1) != hipSuccess) goto done;
    if (hipGetLastError() != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess || ms <= 0.f) goto done;
    *gbps = (copy ? 2.0 : 1.0) * (double)(n16 * 16) * iters / (ms / 1000.0) / 1e9;
    rc = 0;
done:   // releases: a failure here leaves rc as it is
    if (st) (void)hipStreamSynchronize(st);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (st) (void)hipStreamDestroy(st);
    if (a) (void)hipFree(a);
    if (b) (void)hipFree(b);
    if (sink) (void)hipFree(sink);
    return rc;
}

}  // namespace

extern "C" int ccp_read_gbps(int device, size_t bytes, int iters, double* gbps) {
    return run(device, bytes, iters, false, gbps);
}

extern "C" int ccp_copy_gbps(int device, size_t bytes, int iters, double* gbps) {
    return run(device, bytes, iters, true, gbps);
}
