// Stage 1b: block selection at a refresh.
//   block_scores   fp32 S = scale * qbar . kbar (recap/sparse/router.py:18-19); every score
//                  is a sequential sum over channels of separately rounded products (no
//                  FMA contraction), then one rounded multiply by fp32(scale), so the
//                  masks are reproducible bit for bit.
//   topk           top-`keep` key blocks per query block (recap/sparse/router.py:20-22),
//                  ties to the lower block index, plus the forced trailing partial block
//                  (recap/sparse/attention.py:88-94); one workgroup per row, bitonic sort
//                  of (monotone score key, index) pairs in LDS.
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

constexpr int kMaxSortBlocks = 4096;

__global__ __launch_bounds__(256) void topk_kernel(TopkArgs a) {
  __shared__ unsigned long long key[kMaxSortBlocks];
  __shared__ uint8_t sel[kMaxSortBlocks];
  const int row = blockIdx.x % a.nb, bank = blockIdx.x / a.nb;
  const int t = threadIdx.x;
  const float* s = a.scores + ((int64_t)bank * a.nb + row) * a.nb;
  int P = 1;
  while (P < a.nb) P <<= 1;
  for (int j = t; j < P; j += 256) {
    unsigned long long k = 0ull;
    if (j < a.nb) {
      const unsigned bits = __float_as_uint(s[j]);
      const unsigned mono = (bits >> 31) ? ~bits : (bits | 0x80000000u);
      k = ((unsigned long long)mono << 32) | (unsigned long long)(0xffffffffu - (unsigned)j);
    }
    key[j] = k;
    sel[j] = 0;
  }
  __syncthreads();
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = t; i < P; i += 256) {
        const int p = i ^ stride;
        if (p > i) {
          const unsigned long long x = key[i], y = key[p];
          const bool desc = (i & size) == 0;
          if (desc ? (x < y) : (x > y)) { key[i] = y; key[p] = x; }
        }
      }
      __syncthreads();
    }
  }
  for (int i = t; i < a.keep; i += 256) {
    sel[0xffffffffu - (unsigned)(key[i] & 0xffffffffull)] = 1;
  }
  __syncthreads();
  uint8_t* out = a.partition + ((int64_t)bank * a.nb + row) * a.nb;
  const bool full_row = a.force_last && row == a.nb - 1;
  for (int j = t; j < a.nb; j += 256) {
    out[j] = (sel[j] || full_row || (a.force_last && j == a.nb - 1)) ? 1 : 0;
  }
}

hipError_t run_topk(const TopkArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(topk_kernel, dim3((unsigned)(a.banks * a.nb)), dim3(256), 0, s, a);
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

__global__ __launch_bounds__(256) void overlap_partial_kernel(const uint8_t* a, const uint8_t* b,
                                                              int64_t n,
                                                              unsigned long long* part) {
  __shared__ unsigned long long sk[256], st[256];
  unsigned long long kept = 0, total = 0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256) {
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
