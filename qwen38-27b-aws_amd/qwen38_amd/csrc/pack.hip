// Weight packing: FP8 e4m3 bytes [N][K] and E8M0 scale bytes [N][K/32] (row per output feature) into the tiles the
// GEMMs read (common.h): tile (n / 32, k / 64) of 2 KiB as [m][lane][8], lane (n % 32) + 32 * h holding inputs
// 32 * (m / 2) + 16 * h + 8 * (m % 2) + [0, 8) of the K-step at step m; and per tile 64 scale bytes [row][block],
// block 0 scaling the K-step's inputs [0, 32) (steps 0-1), block 1 inputs [32, 64) (steps 2-3).
#include "kernels.h"

__global__ void pack_tiles_kernel(const uint8_t* coded, int N, int K, uint8_t* tiles) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // 8-byte chunk of the output
    if (i >= (size_t)N * K / 8) return;
    const int KS = K >> 6;
    const size_t tile = i >> 8;
    const int m = (int)((i >> 6) & 3), lane = (int)(i & 63);
    const int nt = (int)(tile / KS), ks = (int)(tile % KS);
    const int n = nt * 32 + (lane & 31), k = ks * 64 + 32 * (m >> 1) + 16 * (lane >> 5) + 8 * (m & 1);
    *(uint2*)(tiles + i * 8) = *(const uint2*)(coded + (size_t)n * K + k);
}

__global__ void pack_scales_kernel(const uint8_t* scales, int N, int K, uint8_t* out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // output byte
    const int KS = K >> 6;
    if (i >= (size_t)N * KS * 2) return;
    const int b = (int)(i & 1), r = (int)((i >> 1) & 31);
    const size_t tile = i >> 6;
    const int nt = (int)(tile / KS), ks = (int)(tile % KS);
    out[i] = scales[(size_t)(nt * 32 + r) * (K / 32) + ks * 2 + b];
}

// MXFP4 weights (the checkpoint's bytes [N][K/2], the even input in the low nibble) into tiles of 1 KiB with the same
// element order: 4 bytes per lane and step, the 8 inputs of the step in order (a contiguous 4-byte run of the row).
__global__ void pack_tiles_fp4_kernel(const uint8_t* packed, int N, int K, uint8_t* tiles) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // 4-byte chunk of the output
    if (i >= (size_t)N * K / 8) return;
    const int KS = K >> 6;
    const size_t tile = i >> 8;
    const int m = (int)((i >> 6) & 3), lane = (int)(i & 63);
    const int nt = (int)(tile / KS), ks = (int)(tile % KS);
    const int n = nt * 32 + (lane & 31), k = ks * 64 + 32 * (m >> 1) + 16 * (lane >> 5) + 8 * (m & 1);
    *(uint32_t*)(tiles + i * 4) = *(const uint32_t*)(packed + (size_t)n * (K / 2) + k / 2);
}

hipError_t q38_pack_fp4(const uint8_t* packed, const uint8_t* scales, int N, int K, uint8_t* tiles, uint8_t* tile_scales,
                        hipStream_t stream) {
    size_t chunks = (size_t)N * K / 8;
    hipLaunchKernelGGL(pack_tiles_fp4_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream, packed, N, K, tiles);
    size_t nbytes = (size_t)N * K / 32;
    hipLaunchKernelGGL(pack_scales_kernel, dim3((unsigned)((nbytes + 255) / 256)), dim3(256), 0, stream, scales, N, K,
                       tile_scales);
    return hipGetLastError();
}

hipError_t q38_pack(const uint8_t* coded, const uint8_t* scales, int N, int K, uint8_t* tiles, uint8_t* tile_scales,
                    hipStream_t stream) {
    size_t chunks = (size_t)N * K / 8;
    hipLaunchKernelGGL(pack_tiles_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream, coded, N, K, tiles);
    size_t nbytes = (size_t)N * K / 32;
    hipLaunchKernelGGL(pack_scales_kernel, dim3((unsigned)((nbytes + 255) / 256)), dim3(256), 0, stream, scales, N, K,
                       tile_scales);
    return hipGetLastError();
}
