// Stage 1b: block selection at a refresh.
//   block_scores   fp32 S = scale * qbar . kbar (recap/sparse/router.py:18-19); every score
//                  is a sequential sum over channels of separately rounded products (no
//                  FMA contraction), then one rounded multiply by fp32(scale), so the
//                  masks are reproducible bit for bit.
//   topk           top-`keep` key blocks per query block (recap/sparse/router.py:20-22),
//                  ties to the lower block index, plus the forced trailing partial block
//                  (recap/sparse/attention.py:88-94); a radix select per row, one wave.
//   kernel_mask    video partition embedded in the kernel's block grid with every row and
//                  column from the dense start on (recap/kernels/block_sparse.py:52-75).
//   mask_overlap   |P_new & P_old| and |P_new| for the rerank decision
//                  (recap/operator.py:423-428); integer counts, exact.
#include "kernels.hpp"

namespace recap {

template <int D>
__global__ __launch_bounds__(256) void block_scores_kernel(ScoreArgs a) {
#pragma clang fp contract(off)
  __shared__ float qs[64][D + 1];
  __shared__ float ks[64][D + 1];
  const int bank = blockIdx.z, i0 = blockIdx.y * 64, j0 = blockIdx.x * 64;
  const int t = threadIdx.x;
  const float* qm = a.qm + (int64_t)bank * a.nb * D;
  const float* km = a.km + (int64_t)bank * a.nb * D;
  for (int idx = t; idx < 64 * D; idx += 256) {
    const int r = idx / D, c = idx % D;
    qs[r][c] = (i0 + r < a.nb) ? qm[(int64_t)(i0 + r) * D + c] : 0.0f;
    ks[r][c] = (j0 + r < a.nb) ? km[(int64_t)(j0 + r) * D + c] : 0.0f;
  }
  __syncthreads();
  const int ty = t >> 4, tx = t & 15;
  float acc[4][4];
#pragma unroll
  for (int ai = 0; ai < 4; ++ai)
#pragma unroll
    for (int bj = 0; bj < 4; ++bj) acc[ai][bj] = qs[ty + 16 * ai][0] * ks[tx + 16 * bj][0];
  for (int c = 1; c < D; ++c) {
    float qv[4], kv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) { qv[i] = qs[ty + 16 * i][c]; kv[i] = ks[tx + 16 * i][c]; }
#pragma unroll
    for (int ai = 0; ai < 4; ++ai)
#pragma unroll
      for (int bj = 0; bj < 4; ++bj) acc[ai][bj] = acc[ai][bj] + qv[ai] * kv[bj];  // two roundings (contract off)
  }
  float* out = a.scores + (int64_t)bank * a.nb * a.nb;
#pragma unroll
  for (int ai = 0; ai < 4; ++ai) {
    const int i = i0 + ty + 16 * ai;
#pragma unroll
    for (int bj = 0; bj < 4; ++bj) {
      const int j = j0 + tx + 16 * bj;
      if (i < a.nb && j < a.nb) out[(int64_t)i * a.nb + j] = acc[ai][bj] * a.scale;
    }
  }
}

hipError_t run_block_scores(const ScoreArgs& a, hipStream_t s) {
  const dim3 grid((a.nb + 63) / 64, (a.nb + 63) / 64, a.banks), block(256);
  if (a.dim == 128) hipLaunchKernelGGL(block_scores_kernel<128>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(block_scores_kernel<64>, grid, block, 0, s, a);
  return hipGetLastError();
}

// Top-k by radix select, one wave per row.  Scores become order-preserving 32-bit keys
// (flip all bits of a negative float, set the sign bit of a positive one); four passes over
// the 8-bit digits from the most significant down find the key T of the keep-th largest
// score exactly: each pass histograms, in LDS, the digit of the keys that match the digits
// fixed so far, and a wave-wide suffix scan over the 256 buckets picks the digit whose
// bucket holds the keep-th key.  The row then takes every key above T and, of the keys equal
// to T, as many as are still needed in ascending block order (ties to the lower index),
// counted with one ballot per 64 blocks.  A row of nb scores is read once and its partition
// row written once; the keys stay in registers (PER per lane).
constexpr int kMaxSortBlocks = 4096;
constexpr int kTopkWaves = 4;

__device__ inline unsigned order_key(float x) {
  const unsigned bits = __float_as_uint(x);
  return (bits >> 31) ? ~bits : (bits | 0x80000000u);
}

template <int PER>
__global__ __launch_bounds__(64 * kTopkWaves) void topk_kernel(TopkArgs a) {
  __shared__ unsigned hist[kTopkWaves][256];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t rows = (int64_t)a.banks * a.nb;
  const int64_t row_id = (int64_t)blockIdx.x * kTopkWaves + wave;
  const bool live = row_id < rows;        // a wave past the last row counts nothing
  const int nb = a.nb;
  const float* s = a.scores + (live ? row_id : 0) * nb;
  unsigned key[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int j = lane + 64 * i;
    key[i] = (live && j < nb) ? order_key(s[j]) : 0u;
  }
  unsigned* h = hist[wave];
  unsigned prefix = 0, fixed = 0;   // digits found so far, and their bit mask
  int need = a.keep;                // keys still to take at or below the current prefix
  for (int shift = 24; shift >= 0; shift -= 8) {
#pragma unroll
    for (int b = lane; b < 256; b += 64) h[b] = 0u;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int j = lane + 64 * i;
      if (live && j < nb && (key[i] & fixed) == prefix) atomicAdd(&h[(key[i] >> shift) & 255], 1u);
    }
    __syncthreads();
    // Lane l owns buckets 255-4l .. 252-4l (descending digits); scan the lanes in order.
    unsigned c[4], own = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) { c[k] = h[255 - 4 * lane - k]; own += c[k]; }
    unsigned above = own;   // inclusive prefix over lanes 0..lane
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const unsigned v = __shfl_up(above, off, 64);
      if (lane >= off) above += v;
    }
    above -= own;           // keys in buckets above this lane's
    int digit = -1;
    unsigned before = above;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (digit < 0 && before < (unsigned)need && (unsigned)need <= before + c[k]) {
        digit = 255 - 4 * lane - k;
        above = before;
      }
      before += c[k];
    }
    // Exactly one bucket holds the keep-th key (none in a wave past the last row).
    const unsigned long long owner = __ballot(digit >= 0);
    const int src = owner ? __ffsll((long long)owner) - 1 : 0;
    digit = owner ? __shfl(digit, src, 64) : 0;
    above = owner ? __shfl(above, src, 64) : 0u;
    prefix |= (unsigned)digit << shift;
    fixed |= 0xffu << shift;
    need -= (int)above;
    __syncthreads();   // the histogram is read by every lane before the next pass clears it
  }
  // prefix is now the keep-th largest key; `need` keys equal to it are taken, lowest first.
  const unsigned long long below = lane ? (~0ull >> (64 - lane)) : 0ull;
  const int row = (int)(row_id % nb);
  const bool full_row = a.force_last && row == nb - 1;
  uint8_t* out = a.partition + (live ? row_id : 0) * nb;
  int taken = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int j = lane + 64 * i;
    const bool valid = live && j < nb;
    const bool tie = valid && key[i] == prefix;
    const unsigned long long ties = __ballot(tie);
    const bool pick = valid && (key[i] > prefix || (tie && taken + __popcll(ties & below) < need));
    taken += __popcll(ties);
    if (valid) out[j] = (pick || full_row || (a.force_last && j == nb - 1)) ? 1 : 0;
  }
}

hipError_t run_topk(const TopkArgs& a, hipStream_t s) {
  const int64_t rows = (int64_t)a.banks * a.nb;
  const dim3 grid((unsigned)((rows + kTopkWaves - 1) / kTopkWaves)), block(64 * kTopkWaves);
  if (a.nb <= 256) hipLaunchKernelGGL(topk_kernel<4>, grid, block, 0, s, a);
  else if (a.nb <= 1024) hipLaunchKernelGGL(topk_kernel<16>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(topk_kernel<kMaxSortBlocks / 64>, grid, block, 0, s, a);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void kernel_mask_kernel(KmaskArgs a) {
  const int64_t total = (int64_t)a.banks * a.tb * a.tb;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * 256) {
    const int j = (int)(idx % a.tb);
    const int i = (int)((idx / a.tb) % a.tb);
    const int64_t bank = idx / ((int64_t)a.tb * a.tb);
    uint8_t v = 1;
    if (i < a.ds && j < a.ds) v = a.partition[(bank * a.nb + i) * a.nb + j] ? 1 : 0;
    a.kmask[idx] = v;
  }
}

hipError_t run_kernel_mask(const KmaskArgs& a, hipStream_t s) {
  const int64_t total = (int64_t)a.banks * a.tb * a.tb;
  const int64_t want = (total + 255) / 256;
  const unsigned blocks = (unsigned)(want < 4096 ? want : 4096);
  hipLaunchKernelGGL(kernel_mask_kernel, dim3(blocks), dim3(256), 0, s, a);
  return hipGetLastError();
}

constexpr int kOverlapBlocks = 256;

// Partition bytes are 0 or 1, so a 32-bit word's set bytes are its popcount: 16 bytes per
// thread and load when both masks are 16-byte aligned, one byte at a time for the rest.
__global__ __launch_bounds__(256) void overlap_partial_kernel(const uint8_t* a, const uint8_t* b,
                                                              int64_t n,
                                                              unsigned long long* part) {
  __shared__ unsigned long long sk[256], st[256];
  unsigned long long kept = 0, total = 0;
  const int64_t stride = (int64_t)gridDim.x * 256;
  const int64_t first = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const bool wide = ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15) == 0;
  const int64_t n16 = wide ? n / 16 : 0;
  for (int64_t i = first; i < n16; i += stride) {
    const u32x4 x = reinterpret_cast<const u32x4*>(a)[i];
    const u32x4 y = reinterpret_cast<const u32x4*>(b)[i];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      total += __builtin_popcount(x[w]);
      kept += __builtin_popcount(x[w] & y[w]);
    }
  }
  for (int64_t i = 16 * n16 + first; i < n; i += stride) {
    const bool x = a[i] != 0;
    total += x;
    kept += x && (b[i] != 0);
  }
  sk[threadIdx.x] = kept;
  st[threadIdx.x] = total;
  __syncthreads();
  for (int h = 128; h >= 1; h >>= 1) {
    if ((int)threadIdx.x < h) {
      sk[threadIdx.x] += sk[threadIdx.x + h];
      st[threadIdx.x] += st[threadIdx.x + h];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    part[2 + 2 * blockIdx.x] = sk[0];
    part[3 + 2 * blockIdx.x] = st[0];
  }
}

__global__ void overlap_final_kernel(unsigned long long* part) {
  if (threadIdx.x == 0) {
    unsigned long long k = 0, t = 0;
    for (int i = 0; i < kOverlapBlocks; ++i) { k += part[2 + 2 * i]; t += part[3 + 2 * i]; }
    part[0] = k;
    part[1] = t;
  }
}

// out: [2 + 2*kOverlapBlocks] u64; out[0] = |a & b|, out[1] = |a|.
hipError_t run_mask_overlap(const uint8_t* a, const uint8_t* b, int64_t n, unsigned long long* out,
                            hipStream_t s) {
  hipLaunchKernelGGL(overlap_partial_kernel, dim3(kOverlapBlocks), dim3(256), 0, s, a, b, n, out);
  hipLaunchKernelGGL(overlap_final_kernel, dim3(1), dim3(64), 0, s, out);
  return hipGetLastError();
}

}  // namespace recap
