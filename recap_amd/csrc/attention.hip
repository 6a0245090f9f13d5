// Stage 2: block-sparse flash attention on bf16/fp16 MFMA (v_mfma_f32_32x32x16_*).
//
// Exact softmax attention of each 128-row query block over the key blocks its row of the
// kernel mask selects, with natural-log LSE -- the semantics of the external
// block_sparse_attn_func call at recap/kernels/block_sparse.py:111-138.  Same kernel, all
// blocks kept, is the dense attention + LSE of a refresh (recap/operator.py:254-256).
//
// Workgroup = one (bank, query block): 4 waves x 32 query rows.  Each wave computes
// S^T = K Q^T (keys x queries) so that a lane owns one query row: the row max needs one
// lane-pair exchange per key tile and the row sum none until the end.  The fp32 S^T
// registers become the B operand P^T of O^T = V^T P^T directly; the packed V^T tile stores
// its keys in the matching order (swap23), so no shuffle is needed.  K and V^T tiles are
// verbatim images in HBM (written once per call by pack_pool) copied into XOR-swizzled
// LDS.  Q rows and the output rows go through the Hilbert row map, i.e. the reorder and
// restore of recap/operator.py:496-498, 527 are fused into the loads and stores.
//
// Epilogues:
//   head   (oh fp32, lh) in reordered order -- the head branch a refresh capture needs;
//   dense  output + LSE in native order -- a refresh's dense call;
//   merge  head (+) [coarse tail + drift-weighted refinement] in LSE space for rows < R,
//          the head alone above (recap/kernels/detail_cache.py:220-301), written in
//          native order: the whole corrected sparse output in one pass.
#include <type_traits>

#include "kernels.hpp"

namespace recap {

constexpr int kMaxTiles = 2048;

// Rows whose running max grows by less than this (log2 units) keep their stale max: p then
// stays below 2^8, exact in fp32 and bf16, and the O rescale is skipped.
constexpr float kRescaleSlack = 8.0f;

template <class T, int D, int MODE>
__global__ __launch_bounds__(256, 2) void attention_kernel(AttnArgs a) {
  using G = TileGeom<D>;
  constexpr int NS = D / 16;                  // k-steps over the head dimension
  constexpr int NDT = D / 32;                 // 32-row tiles of O^T
  constexpr int HALF = G::kHalfBytes;         // K or V^T part of a 64-key sub-tile
  constexpr int SUB = 2 * HALF;               // one sub-tile image in LDS
  constexpr int NLD = SUB / 16 / 256;         // 16-byte loads per thread per sub-tile
  __shared__ __attribute__((aligned(16))) char lds[2 * SUB];
  __shared__ int list[MODE == kModeDense ? 1 : kMaxTiles];
  __shared__ int scan[256];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, g = lane >> 5, l32 = lane & 31;
  // Bank-major order across all XCDs (workgroup i runs on XCD i % 8): the workgroups in
  // flight cover one or two banks, whose K/V tiles (61 MB per bank at the HunyuanVideo
  // shape) then stay resident in the 256 MB Infinity Cache.
  const int lin = blockIdx.x;
  const int bank = lin / a.tb;
  const int k_in_bank = lin % a.tb;
  const int ndense = a.tb - a.ds;  // dense query blocks first: they are the longest
  const int qt = k_in_bank < ndense ? a.ds + k_in_bank : k_in_bank - ndense;
  const int b = bank / a.heads, h = bank % a.heads;

  int nkeep = a.tb;
  if constexpr (MODE != kModeDense) {
    const uint8_t* mrow = a.kmask + ((int64_t)bank * a.tb + qt) * a.tb;
    const int per = (a.tb + 255) / 256;
    const int j0 = min(t * per, a.tb), j1 = min(j0 + per, a.tb);
    int cnt = 0;
    for (int j = j0; j < j1; ++j) cnt += mrow[j] != 0;
    scan[t] = cnt;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
      const int v = t >= off ? scan[t - off] : 0;
      __syncthreads();
      scan[t] += v;
      __syncthreads();
    }
    int pos = scan[t] - cnt;
    for (int j = j0; j < j1; ++j)
      if (mrow[j]) list[pos++] = j;
    nkeep = scan[255];
    __syncthreads();
  }
  const int nsub = 2 * nkeep;  // 64-key sub-tiles

  // Sub-tile `it` = half (it & 1) of kept tile (it >> 1): its K rows and its V^T half are
  // each HALF contiguous bytes of the packed images.
  u32x4 pre[NLD];
  auto fetch = [&](int it) {
    const int j = MODE == kModeDense ? (it >> 1) : list[it >> 1];
    const int64_t tile = ((int64_t)bank * a.tb + j) * G::kTileElems;
    const u32x4* ks = reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(a.kp + tile) + (it & 1) * HALF);
    const u32x4* vs = reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(a.vp + tile) + (it & 1) * HALF);
#pragma unroll
    for (int i = 0; i < NLD / 2; ++i) {
      pre[i] = ks[t + 256 * i];
      pre[NLD / 2 + i] = vs[t + 256 * i];
    }
  };
  auto stash = [&](int buf) {
    u32x4* dst = reinterpret_cast<u32x4*>(lds + buf * SUB);
#pragma unroll
    for (int i = 0; i < NLD / 2; ++i) {
      dst[t + 256 * i] = pre[i];
      dst[HALF / 16 + t + 256 * i] = pre[NLD / 2 + i];
    }
  };

  const int r = qt * kBlock + wave * 32 + l32;
  const bool rv = r < a.n_tokens;
  const int nat = rv ? a.rowmap[r] : 0;
  if (nsub > 0) fetch(0);
  u32x4 qreg[NS];
  {
    const uint16_t* qrow = a.q + b * a.qsB + h * a.qsH + (int64_t)nat * a.qsN;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      qreg[s] = rv ? *reinterpret_cast<const u32x4*>(qrow + 16 * s + 8 * g) : u32x4{0u, 0u, 0u, 0u};
    }
  }
  if (nsub > 0) stash(0);
  if (nsub > 1) fetch(1);
  __syncthreads();

  float m = -INFINITY, lsum = 0.0f;
  f32x16 oacc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) oacc[dt] = f32x16{};
  const bool ragged = (a.n_tokens % kBlock) != 0;

  auto step = [&](int it, auto ragged_tag) {
    constexpr bool kRagged = decltype(ragged_tag)::value;
    const char* k_lds = lds + (it & 1) * SUB;
    const char* v_lds = k_lds + HALF;

    f32x16 sacc[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      sacc[kt] = f32x16{};
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const u32x4 ka = lds_load16(k_lds, G::k_off(32 * kt + l32, 2 * s + g));
        sacc[kt] = T::mfma32(ka, qreg[s], sacc[kt]);
      }
    }
    if constexpr (kRagged) {
      const int limit = a.n_tokens - ((a.tb - 1) * kBlock + 64 * (it & 1));
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int rr = 0; rr < 16; ++rr)
          if (32 * kt + mfma_row(rr, g) >= limit) sacc[kt][rr] = -INFINITY;
    }

    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) mx = fmaxf(mx, sacc[kt][rr]);
    const float mt = pair_max(mx) * a.scale_log2;
    const bool grow = mt > m + kRescaleSlack;
    if (__any(grow)) {
      const float mnew = grow ? mt : m;
      const float alpha = __builtin_amdgcn_exp2f(m - mnew);
      lsum *= alpha;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) oacc[dt] *= alpha;
      m = mnew;
    }

    u32x4 pk[2][2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        unsigned w[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const float p0 = __builtin_amdgcn_exp2f(fmaf(sacc[kt][8 * hh + e], a.scale_log2, -m));
          const float p1 = __builtin_amdgcn_exp2f(fmaf(sacc[kt][8 * hh + e + 1], a.scale_log2, -m));
          lsum += p0 + p1;
          w[e >> 1] = pack2<T>(p0, p1);
        }
        pk[kt][hh] = u32x4{w[0], w[1], w[2], w[3]};
      }
    }
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const u32x4 va = lds_load16(v_lds, G::vt_off(32 * dt + l32, 4 * kt + 2 * hh + g));
          oacc[dt] = T::mfma32(va, pk[kt][hh], oacc[dt]);
        }
      }
    }

    // Sub-tile it+1 (fetched during this one) goes to the other buffer, whose last reader
    // was iteration it-1; then fetch it+2 and wait for everyone.
    if (it + 1 < nsub) stash((it + 1) & 1);
    if (it + 2 < nsub) fetch(it + 2);
    __syncthreads();
  };
  // The last kept tile holds the ragged keys when it is the sequence's last block.
  const bool ragged_last = ragged && nkeep > 0 &&
                           (MODE == kModeDense ? true : list[nkeep - 1] == a.tb - 1);
  const int plain = ragged_last ? nsub - 2 : nsub;
  for (int it = 0; it < plain; ++it) step(it, std::false_type{});
  for (int it = plain; it < nsub; ++it) step(it, std::true_type{});

  if (!rv) return;
  const float lt = pair_sum(lsum);
  const float inv = 1.0f / lt;
  const float lse = (m + log2f(lt)) * kLn2;

  if constexpr (MODE == kModeHead) {
    // fp32 head branch: the capture and the merge then see the same unrounded values.
    float* orow = a.head_out + ((int64_t)bank * a.n_tokens + r) * D;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d0 = 32 * dt + 8 * q4 + 4 * g;
        *reinterpret_cast<f32x4*>(orow + d0) =
            f32x4{oacc[dt][4 * q4] * inv, oacc[dt][4 * q4 + 1] * inv,
                  oacc[dt][4 * q4 + 2] * inv, oacc[dt][4 * q4 + 3] * inv};
      }
    if (g == 0) a.head_lse[(int64_t)bank * a.n_tokens + r] = lse;
    return;
  }

  uint16_t* orow = a.out + b * a.osB + h * a.osH + (int64_t)nat * a.osN;
  if constexpr (MODE == kModeDense) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d0 = 32 * dt + 8 * q4 + 4 * g;
        u32x2 v = {pack2<T>(oacc[dt][4 * q4] * inv, oacc[dt][4 * q4 + 1] * inv),
                   pack2<T>(oacc[dt][4 * q4 + 2] * inv, oacc[dt][4 * q4 + 3] * inv)};
        *reinterpret_cast<u32x2*>(orow + d0) = v;
      }
    if (g == 0) a.lse_native[(int64_t)bank * a.n_tokens + nat] = lse;
    return;
  }

  // Merge epilogue (recap/kernels/detail_cache.py:228-301): rows < R get the drift-weighted
  // tail.  The head output is never materialised here, so it enters in fp32 (the reference
  // rounds it to bf16 only because its attention kernel stores a bf16 tensor).
  if (r < a.rows) {
    const int64_t ri = (int64_t)bank * a.rows + r;
    const float glv = a.gl[ri], dlv = a.dl[ri];
    const float admit = a.use_override ? a.alpha_override
                                       : expf(-fabsf(glv - a.glref[ri] - a.center[bank]));
    const float cl = glv + dlv;
    const float tc = fmaxf(glv, cl);
    const float sm = (1.0f - admit) * expf(glv - tc);
    const float cm = admit * expf(cl - tc);
    const float den = fmaxf(sm + cm, 1.0e-30f);
    const float tl = tc + logf(den);
    const float common = fmaxf(lse, tl);
    const float wh = expf(lse - common);
    const float wt = expf(tl - common);
    const float den2 = fmaxf(wh + wt, 1.0e-30f);
    const uint16_t* gorow = a.go + ri * D;
    const uint16_t* drow = a.det + ri * D;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d0 = 32 * dt + 8 * q4 + 4 * g;
        const u32x2 gw = *reinterpret_cast<const u32x2*>(gorow + d0);
        const u32x2 dw = *reinterpret_cast<const u32x2*>(drow + d0);
        float res[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const unsigned gword = gw[e >> 1], dword = dw[e >> 1];
          const float gov = T::to_f((uint16_t)((e & 1) ? gword >> 16 : gword & 0xffff));
          const float detv = f16_to_f((uint16_t)((e & 1) ? dword >> 16 : dword & 0xffff));
          const float ohv = oacc[dt][4 * q4 + e] * inv;
          const float to = (gov * sm + (gov + detv) * cm) / den;
          res[e] = (ohv * wh + to * wt) / den2;
        }
        u32x2 v = {pack2<T>(res[0], res[1]), pack2<T>(res[2], res[3])};
        *reinterpret_cast<u32x2*>(orow + d0) = v;
      }
  } else {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d0 = 32 * dt + 8 * q4 + 4 * g;
        u32x2 v = {pack2<T>(oacc[dt][4 * q4] * inv, oacc[dt][4 * q4 + 1] * inv),
                   pack2<T>(oacc[dt][4 * q4 + 2] * inv, oacc[dt][4 * q4 + 3] * inv)};
        *reinterpret_cast<u32x2*>(orow + d0) = v;
      }
  }
}

template <class T, int D>
static hipError_t launch_attention(const AttnArgs& a, int mode, hipStream_t s) {
  const dim3 grid((unsigned)(a.banks * a.tb)), block(256);
  switch (mode) {
    case kModeHead: hipLaunchKernelGGL((attention_kernel<T, D, kModeHead>), grid, block, 0, s, a); break;
    case kModeDense: hipLaunchKernelGGL((attention_kernel<T, D, kModeDense>), grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL((attention_kernel<T, D, kModeMerge>), grid, block, 0, s, a); break;
  }
  return hipGetLastError();
}

hipError_t run_attention(const AttnArgs& a, int dtype, int dim, int mode, hipStream_t s) {
  if (dtype == BF16::code)
    return dim == 128 ? launch_attention<BF16, 128>(a, mode, s) : launch_attention<BF16, 64>(a, mode, s);
  return dim == 128 ? launch_attention<F16, 128>(a, mode, s) : launch_attention<F16, 64>(a, mode, s);
}

}  // namespace recap
