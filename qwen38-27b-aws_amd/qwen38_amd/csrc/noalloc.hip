// q38_fp8_linear_noalloc: the standalone FP8 projection (q38_fp8_linear) for callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops). Its scratch (the e5m2 input tiles, the stream-K arrival
// counters and partial slots) is this file's static device array instead of a caller's buffer.
//
// Limits: at most 64 rows (decode-sized batches), 64 x k input bytes within 2 MiB (k <= 32768), GPUs of at most 256
// CUs. The array is 66.5 MiB; each GPU the entry point runs on holds its own copy until the process ends. Every call
// on one GPU shares that GPU's array: calls that overlap on one GPU race.

#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "../../../include/q38.h"
#include "kernels.h"

namespace {

constexpr int NOALLOC_ROWS = 64;
constexpr int NOALLOC_CUS = 256;
constexpr size_t NOALLOC_TILES = (size_t)2 << 20;  // e5m2 input tiles: 64 rows x 32768 inputs
constexpr size_t NOALLOC_COUNTERS = (size_t)GEMM_COUNTERS * 8;
// Two partial slots per CU, each the largest workgroup tile the GEMM uses at 64 rows or fewer (512 or 256 features x
// 64 tokens over 8 waves: 32768 floats).
constexpr size_t NOALLOC_FIX_FLOATS = (size_t)2 * NOALLOC_CUS * 32768;
constexpr size_t NOALLOC_BYTES = NOALLOC_TILES + NOALLOC_COUNTERS + NOALLOC_FIX_FLOATS * 4;

static __device__ __align__(256) uint8_t scratch[NOALLOC_BYTES];

// The array's device address on each GPU (host code must not use the array's name: it is a host-side stand-in).
std::mutex g_mutex;
uint8_t* g_scratch[64];

int scratch_on_current_device(uint8_t** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        (void)hipGetLastError();
        return q38_report("q38_fp8_linear_noalloc: no current HIP device");
    }
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!g_scratch[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            return q38_report((std::string("q38_fp8_linear_noalloc: hipGetSymbolAddress(scratch): ") + hipGetErrorString(e)).c_str());
        }
        g_scratch[dev] = (uint8_t*)p;
    }
    *out = g_scratch[dev];
    return 0;
}

__global__ void clear_counters_kernel(unsigned long long* counters, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) counters[i] = 0;
}

}  // namespace

int q38_fp8_linear_noalloc(const uint16_t* x, int rows, int k, const uint8_t* tiles, const uint8_t* tile_scales, int n,
                           uint16_t* out, void* stream_) {
    if (!x || !tiles || !tile_scales || !out) return q38_report("null argument");
    if (rows < 1 || rows > NOALLOC_ROWS) return q38_report("q38_fp8_linear_noalloc takes 1 to 64 rows (its static scratch)");
    if (n < 256 || n % 256 || k < 256 || k % 256) return q38_report("projection needs N % 256 == 0 and K % 256 == 0");
    if (q38_tiles_size(rows, k) > NOALLOC_TILES)
        return q38_report("q38_fp8_linear_noalloc takes K <= 32768 (64 x K input bytes in its static scratch)");
    if (q38_device_cus() > NOALLOC_CUS) return q38_report("q38_fp8_linear_noalloc: its static scratch covers 256 CUs");
    uint8_t* base = nullptr;
    if (scratch_on_current_device(&base)) return 1;
    hipStream_t stream = (hipStream_t)stream_;
    // The arrival counters of every tile this call can use start at zero (tiles of 128 or more features, token blocks
    // of 32 or more), cleared by a kernel on the caller's stream, so a captured call records no memset.
    unsigned long long* counters = (unsigned long long*)(base + NOALLOC_TILES);
    const int used = n / 128 * 2 < GEMM_COUNTERS ? n / 128 * 2 : GEMM_COUNTERS;
    hipLaunchKernelGGL(clear_counters_kernel, dim3((used + 255) / 256), dim3(256), 0, stream, counters, used);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return q38_report((std::string("clear_counters_kernel: ") + hipGetErrorString(e)).c_str());
    return q38_projection(x, rows, k, tiles, tile_scales, n, EPI_BF16, base, base + NOALLOC_TILES, NOALLOC_FIX_FLOATS, out,
                          0, stream, 0, 0, 0);
}
