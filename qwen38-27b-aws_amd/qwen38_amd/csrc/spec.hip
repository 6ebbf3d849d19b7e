// Device-side glue of one speculative step (the reference's Scheduler._verify_step and _mtp_drafts,
// qwen38_inf2/scheduler.py:160-193, 269-301), so the whole step runs on the GPU without host round trips:
//   rope_gather    cos/sin rows of a position table (generate.py:25-31 rotary, precomputed per position)
//   select_rows    out[b] = rows[b, idx[b]]                 (scheduler.py:180, `out[rows, take]`)
//   mtp_followup   [current, 0, ...] rows and [draft, 0, ...] ids for the next MTP call (scheduler.py:188-192)
//   verify_tokens  [last emitted, drafts...] per row          (scheduler.py:283)
//   advance        index <- position, position += accepted  (scheduler.py:296-300)
#include "kernels.h"

// An active row whose K tokens from `base` pass the last usable position (the reference's verify_inputs raises
// ValueError when position + tokens > max_seq_len - 1, generate.py:78-79) sets Q38_STATUS_POSITION in *status; the
// gather itself clamps to the table.
__global__ void rope_gather_kernel(const int* base, int offset, int B, int K, int S, const bf16_t* table, bf16_t* cos,
                                   bf16_t* sin, const float* active, int* status) {
    const int row = blockIdx.x, t = row % K, b = row / K, d = threadIdx.x;  // 64 threads: rotary dims
    if (status && t == 0 && d == 0 && active && active[b] > 0.5f && (base[b] < 0 || base[b] + K > S - 1))
        atomicOr(status, Q38_STATUS_POSITION);
    int p = base[b] + offset + t;
    p = min(max(p, 0), S - 1);
    cos[(size_t)row * 64 + d] = table[((size_t)p * 2 + 0) * 64 + d];
    sin[(size_t)row * 64 + d] = table[((size_t)p * 2 + 1) * 64 + d];
}

__global__ void select_rows_kernel(const bf16_t* rows, const int* idx, int K, int H, bf16_t* out) {
    const int b = blockIdx.x;
    const int i = idx ? min(max(idx[b], 0), K - 1) : 0;  // no index array: the first row
    for (int c = threadIdx.x * 8; c < H; c += blockDim.x * 8)
        *(v4i*)(out + (size_t)b * H + c) = *(const v4i*)(rows + ((size_t)b * K + i) * H + c);
}

__global__ void mtp_followup_kernel(const bf16_t* current, const int* draft, int K, int H, bf16_t* states, int* ids) {
    const int b = blockIdx.x;
    for (int c = threadIdx.x * 8; c < K * H; c += blockDim.x * 8) {
        v4i v = c < H ? *(const v4i*)(current + (size_t)b * H + c) : (v4i){0, 0, 0, 0};
        *(v4i*)(states + (size_t)b * K * H + c) = v;
    }
    if (threadIdx.x < K) ids[b * K + threadIdx.x] = threadIdx.x == 0 ? draft[b] : 0;
}

// ids[b] = [picks[b][match[b]], drafts[b][0..K-2]]; at[b] = index[b] + match[b] + 1 (the first follow-up MTP index).
__global__ void verify_tokens_kernel(const int* picks, const int* match, const int* drafts, int B, int K, int* ids) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    const int m = min(max(match[b], 0), K - 1);
    ids[b * K] = picks[b * K + m];
    for (int j = 1; j < K; ++j) ids[b * K + j] = drafts[b * (K - 1) + j - 1];
}

__global__ void offset_positions_kernel(const int* index, const int* match, int add, int B, int* at) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b < B) at[b] = index[b] + match[b] + 1 + add;
}

__global__ void advance_kernel(int* position, int* index, const int* accepted, int B) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    index[b] = position[b];
    position[b] += accepted[b];
}

__global__ void column_kernel(const int* ids, int K, int B, int j, int* drafts) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b < B) drafts[b * (K - 1) + j] = ids[b];
}

hipError_t q38_rope_gather(const int* base, int offset, int B, int K, int S, const bf16_t* table, bf16_t* cos, bf16_t* sin,
                           hipStream_t s, const float* active, int* status) {
    hipLaunchKernelGGL(rope_gather_kernel, dim3(B * K), dim3(64), 0, s, base, offset, B, K, S, table, cos, sin, active,
                       status);
    return hipGetLastError();
}

hipError_t q38_select_rows(const bf16_t* rows, const int* idx, int B, int K, int H, bf16_t* out, hipStream_t s) {
    hipLaunchKernelGGL(select_rows_kernel, dim3(B), dim3(256), 0, s, rows, idx, K, H, out);
    return hipGetLastError();
}

hipError_t q38_mtp_followup(const bf16_t* current, const int* draft, int B, int K, int H, bf16_t* states, int* ids,
                            hipStream_t s) {
    hipLaunchKernelGGL(mtp_followup_kernel, dim3(B), dim3(256), 0, s, current, draft, K, H, states, ids);
    return hipGetLastError();
}

hipError_t q38_verify_tokens(const int* picks, const int* match, const int* drafts, int B, int K, int* ids, hipStream_t s) {
    hipLaunchKernelGGL(verify_tokens_kernel, dim3((B + 63) / 64), dim3(64), 0, s, picks, match, drafts, B, K, ids);
    return hipGetLastError();
}

hipError_t q38_offset_positions(const int* index, const int* match, int add, int B, int* at, hipStream_t s) {
    hipLaunchKernelGGL(offset_positions_kernel, dim3((B + 63) / 64), dim3(64), 0, s, index, match, add, B, at);
    return hipGetLastError();
}

hipError_t q38_advance(int* position, int* index, const int* accepted, int B, hipStream_t s) {
    hipLaunchKernelGGL(advance_kernel, dim3((B + 63) / 64), dim3(64), 0, s, position, index, accepted, B);
    return hipGetLastError();
}

hipError_t q38_draft_column(const int* ids, int K, int B, int j, int* drafts, hipStream_t s) {
    hipLaunchKernelGGL(column_kernel, dim3((B + 63) / 64), dim3(64), 0, s, ids, K, B, j, drafts);
    return hipGetLastError();
}
