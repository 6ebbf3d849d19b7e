// Weight packing: FP8 e4m3 bytes [N][K] and E8M0 scale bytes [N][K/32] (row per output feature) into the tiles the
// GEMMs read (common.h): tile (n / 32, k / 64) of 2 KiB, lane (n % 32) + 32 * h, with bytes 0-15 = inputs
// [16h, 16h + 16) and bytes 16-31 = inputs [32 + 16h, 32 + 16h + 16) of the K-step; and scale words [N/32][K/256][64]
// whose byte j, in lane half h, is the scale of MX block h of K-step 4q + j (the scale the MFMA takes from that lane).
#include "kernels.h"

__global__ void pack_tiles_kernel(const uint8_t* coded, int N, int K, uint8_t* tiles) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // 16-byte chunk of the output
    const size_t total = (size_t)N * K / 16;
    if (i >= total) return;
    const int KS = K >> 6;
    const size_t tile = i >> 7;
    const int within = (int)(i & 127), lane = within >> 1, half16 = within & 1;
    const int nt = (int)(tile / KS), ks = (int)(tile % KS);
    const int n = nt * 32 + (lane & 31), k = ks * 64 + half16 * 32 + (lane >> 5) * 16;
    *(v4i*)(tiles + i * 16) = *(const v4i*)(coded + (size_t)n * K + k);
}

__global__ void pack_scales_kernel(const uint8_t* scales, int N, int K, uint32_t* words) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int KQ = K >> 8;
    const size_t total = (size_t)(N / 32) * KQ * 64;
    if (i >= total) return;
    const int lane = (int)(i & 63);
    const size_t rest = i >> 6;
    const int kq = (int)(rest % KQ), nt = (int)(rest / KQ);
    const int n = nt * 32 + (lane & 31), half = lane >> 5;
    const uint8_t* row = scales + (size_t)n * (K / 32);
    uint32_t w = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) w |= (uint32_t)row[(4 * kq + j) * 2 + half] << (8 * j);
    words[i] = w;
}

hipError_t q38_pack(const uint8_t* coded, const uint8_t* scales, int N, int K, uint8_t* tiles, uint32_t* words,
                    hipStream_t stream) {
    size_t chunks = (size_t)N * K / 16;
    hipLaunchKernelGGL(pack_tiles_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream, coded, N, K, tiles);
    size_t nwords = (size_t)(N / 32) * (K / 256) * 64;
    hipLaunchKernelGGL(pack_scales_kernel, dim3((unsigned)((nwords + 255) / 256)), dim3(256), 0, stream, scales, N, K, words);
    return hipGetLastError();
}
