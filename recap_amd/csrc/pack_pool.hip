// Stage 1a: one pass over a 128-token block of K and V (or Q) that
//   * gathers the rows through the Hilbert row map (fused Layout.reorder,
//     recap/sparse/layout.py:82-86), so no reordered copy of Q/K/V is ever written;
//   * writes the packed K tile and V^T tile images the attention kernel copies into LDS;
//   * computes the fp32 block means of the video tokens (recap/sparse/pooling.py:10-34)
//     with a fixed reduction order: thread lane rl adds rows rl, rl+RP, ... in order,
//     then the RP lane partials are combined by a halving tree (RP = 2048 / D).
// HBM-bound: every element is read once and written once (packed), 16-byte accesses.
#include "kernels.hpp"

namespace recap {

template <class T, int D, bool PACK>
__global__ __launch_bounds__(256) void pack_pool_kernel(PackPoolArgs a) {
  constexpr int TPR = D / 8;          // threads per 16-element... per row (16 B each)
  constexpr int RP = 256 / TPR;       // row lanes
  constexpr int PASSES = kBlock / RP; // rows per thread
  using G = TileGeom<D>;
  __shared__ float part[RP][D];
  __shared__ uint16_t vstage[PACK ? kBlock : 1][D + 8];

  const int tile = blockIdx.x % a.tb;
  const int bank = blockIdx.x / a.tb;
  const int b = bank / a.heads, h = bank % a.heads;
  const int t = threadIdx.x, cg = t % TPR, rl = t / TPR;
  const bool video_block = tile < a.nb;
  const int count = min(kBlock, a.n_video - tile * kBlock);

  // Every row load of the block is issued before the first store: the stores go to other
  // buffers, but the compiler cannot prove it and would otherwise wait for each load in turn.
  constexpr int NX = PACK ? 2 : 1;
  u32x4 vals[NX][PASSES];
  {
    // Branch-free: rows past the sequence end load row n_tokens - 1 and are zeroed after.
    int64_t nat[PASSES];
    bool live[PASSES];
#pragma unroll
    for (int i = 0; i < PASSES; ++i) {
      const int r = tile * kBlock + rl + RP * i;
      live[i] = r < a.n_tokens;
      nat[i] = a.rowmap[min(r, a.n_tokens - 1)];
    }
#pragma unroll
    for (int which = 0; which < NX; ++which) {
      const uint16_t* src = which == 0 ? a.x0 : a.x1;
      const int64_t sB = which == 0 ? a.sB0 : a.sB1, sH = which == 0 ? a.sH0 : a.sH1,
                    sN = which == 0 ? a.sN0 : a.sN1;
      const uint16_t* base = src + b * sB + h * sH;
#pragma unroll
      for (int i = 0; i < PASSES; ++i) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(base + nat[i] * sN + cg * 8);
        vals[which][i] = live[i] ? v : u32x4{0u, 0u, 0u, 0u};
      }
    }
  }

#pragma unroll
  for (int which = 0; which < NX; ++which) {
    float acc[8];
#pragma unroll
    for (int i = 0; i < PASSES; ++i) {
      const int row = rl + RP * i;
      const int r = tile * kBlock + row;
      const u32x4 val = vals[which][i];
      if constexpr (PACK) {
        if (which == 0) {
          char* dst = reinterpret_cast<char*>(a.kp + ((int64_t)bank * a.tb + tile) * G::kTileElems);
          *reinterpret_cast<u32x4*>(dst + G::k_off(row, cg)) = val;
        } else {
          *reinterpret_cast<u32x4*>(&vstage[row][cg * 8]) = val;
        }
      }
      const bool in_video = r < a.n_video;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const unsigned word = val[e >> 1];
        const uint16_t hv = (e & 1) ? (uint16_t)(word >> 16) : (uint16_t)(word & 0xffff);
        const float x = in_video ? T::to_f(hv) : 0.0f;
        acc[e] = (i == 0) ? x : acc[e] + x;
      }
    }
    if (video_block) {
#pragma unroll
      for (int e = 0; e < 8; ++e) part[rl][cg * 8 + e] = acc[e];
      __syncthreads();
      for (int half = RP / 2; half >= 1; half >>= 1) {
        if (rl < half) {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            part[rl][cg * 8 + e] = part[rl][cg * 8 + e] + part[rl + half][cg * 8 + e];
        }
        __syncthreads();
      }
      float* mean_out = which == 0 ? a.mean0 : a.mean1;
      if (t < D) {
        mean_out[((int64_t)bank * a.nb + tile) * D + t] = __fdiv_rn(part[0][t], (float)count);
      }
    }
    __syncthreads();
  }

  if constexpr (PACK) {
    // V^T image: position p of row d holds key swap23(p).
    char* dst = reinterpret_cast<char*>(a.vp + ((int64_t)bank * a.tb + tile) * G::kTileElems);
    for (int cc = t; cc < D * 16; cc += 256) {
      const int d = cc >> 4, c = cc & 15;
      unsigned w[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const int k0 = swap23(8 * c + e), k1 = swap23(8 * c + e + 1);
        w[e >> 1] = (unsigned)vstage[k0][d] | ((unsigned)vstage[k1][d] << 16);
      }
      u32x4 v = {w[0], w[1], w[2], w[3]};
      *reinterpret_cast<u32x4*>(dst + G::vt_off(d, c)) = v;
    }
  }
}

template <class T, int D>
static hipError_t launch_pack_pool(const PackPoolArgs& a, bool pack, hipStream_t s) {
  const dim3 grid((unsigned)(a.banks * a.tb)), block(256);
  if (pack) hipLaunchKernelGGL((pack_pool_kernel<T, D, true>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((pack_pool_kernel<T, D, false>), grid, block, 0, s, a);
  return hipGetLastError();
}

hipError_t run_pack_pool(const PackPoolArgs& a, int dtype, int dim, bool pack, hipStream_t s) {
  if (dtype == BF16::code) {
    return dim == 128 ? launch_pack_pool<BF16, 128>(a, pack, s) : launch_pack_pool<BF16, 64>(a, pack, s);
  }
  return dim == 128 ? launch_pack_pool<F16, 128>(a, pack, s) : launch_pack_pool<F16, 64>(a, pack, s);
}

}  // namespace recap
