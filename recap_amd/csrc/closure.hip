// Stage 3 prerequisites: the moment statistics of the coarse tail, read from the packed
// K / V^T tiles written by pack_pool.
//   rot      per-block mean and clamped variance of U^T k with U as a hi+lo pair in the
//            input type (recap/kernels/closure_stats.py:96-189, 192-242)
//   cvk      partial sums of V^T (K - kbar_block) with the centred key as a hi+lo pair
//            (recap/kernels/closure_stats.py:27-94, 245-290)
//   scatter  partial sums of the within-block key scatter (K - kbar)^T (K - kbar) as
//            hi.hi + hi.lo + lo.hi (recap/sparse/closure.py:42-72, first call only)
// A workgroup handles `group` consecutive video blocks of one bank and writes one
// [D][D] partial per group; partial_reduce sums the groups in a fixed order and divides
// by the video token count.  tables builds the query-type tables of the coarse tail
// (fold_rank of recap/sparse/closure.py:96-104; kbar, vbar, w casts of
// recap/kernels/coarse_tail.py:238-241) and basis_tables the U / C_vk casts.
#include "kernels.hpp"

namespace recap {

// Threads of a closure workgroup.  The per-call statistics at d = 128 (rotated moments and
// C_vk) split the work by wave: waves 0-3 the rotation, waves 4-7 C_vk, so each wave holds
// one job's registers and every SIMD runs two waves whose MFMA and VALU phases interleave.
// Otherwise four waves each take one 32-row tile of every job.
constexpr int closure_threads(int D, int FLAGS) {
  return D == 128 && FLAGS == (kRot | kCvk) ? 512 : 256;
}

template <class T, int D, int FLAGS>
__global__ __launch_bounds__(closure_threads(D, FLAGS), 1) void closure_kernel(ClosureArgs a) {
  using G = TileGeom<D>;
  constexpr int NS = D / 16, NT = D / 32;
  constexpr bool ROT = (FLAGS & kRot) != 0, CVK = (FLAGS & kCvk) != 0, SCAT = (FLAGS & kScatter) != 0;
  constexpr int NTHR = closure_threads(D, FLAGS);
  constexpr bool SPLIT = NTHR == 512;
  constexpr bool KC = SCAT;  // centred keys staged in LDS (the scatter's A and B operands)
  __shared__ __attribute__((aligned(16))) char k_lds[G::kTileBytes];
  __shared__ __attribute__((aligned(16))) char v_lds[CVK ? G::kTileBytes : 16];
  __shared__ __attribute__((aligned(16))) char kc_hi[KC ? D * 256 : 16];
  __shared__ __attribute__((aligned(16))) char kc_lo[KC ? D * 256 : 16];
  __shared__ float kmean_s[D];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, g = lane >> 5, l32 = lane & 31;
  const int bank = blockIdx.x / a.groups, grp = blockIdx.x % a.groups;
  const int j0 = grp * a.group, j1 = min(j0 + a.group, a.nb);
  const int rot_tile = SPLIT ? (wave < 4 ? wave : -1) : D == 128 ? wave : (wave < 2 ? wave : -1);
  const int mat_tile = SPLIT ? (wave >= 4 ? wave - 4 : -1)
                             : D == 128 ? wave : (wave >= 2 ? wave - 2 : -1);

  // Registers that persist across blocks: a rotation wave's U^T hi/lo fragments (2 NS
  // u32x4) and a C_vk wave's accumulators (NT f32x16).  In the split layout a wave has one
  // job, never both, so the two share one array (64 registers at d = 128).
  struct Quad { u32x4 v[4]; };
  static_assert(!SPLIT || 2 * NS == 4 * NT, "shared persistent registers");
  u32x4 ub[SPLIT ? 2 * NS : (ROT ? 2 * NS : 1)];
  f32x16 cacc_own[!SPLIT && CVK ? NT : 1];
  auto cget = [&](int mt) -> f32x16 {
    if constexpr (SPLIT)
      return __builtin_bit_cast(f32x16, Quad{{ub[4 * mt], ub[4 * mt + 1], ub[4 * mt + 2], ub[4 * mt + 3]}});
    else
      return cacc_own[mt];
  };
  auto cset = [&](int mt, f32x16 v) {
    if constexpr (SPLIT) {
      const Quad q = __builtin_bit_cast(Quad, v);
#pragma unroll
      for (int i = 0; i < 4; ++i) ub[4 * mt + i] = q.v[i];
    } else {
      cacc_own[mt] = v;
    }
  };
  if constexpr (ROT) {
    if (rot_tile >= 0) {
      const int o = 32 * rot_tile + l32;
      const uint16_t* hi = a.u_hi_t + ((int64_t)bank * D + o) * D;
      const uint16_t* lo = a.u_lo_t + ((int64_t)bank * D + o) * D;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        ub[s] = *reinterpret_cast<const u32x4*>(hi + 16 * s + 8 * g);
        ub[NS + s] = *reinterpret_cast<const u32x4*>(lo + 16 * s + 8 * g);
      }
    }
  }
  // Identity slices for the centred-key product: B operand hh holds 1 where key-dimension
  // 16 hh + 8 g + e equals this lane's column l32 (e = 0..7), 0 elsewhere.
  u32x4 bid[2];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int e = l32 - 16 * hh - 8 * g;
    const unsigned one = (T::code == BF16::code ? 0x3f80u : 0x3c00u) << (16 * (e & 1));
    bid[hh] = u32x4{e >> 1 == 0 ? one : 0u, e >> 1 == 1 ? one : 0u, e >> 1 == 2 ? one : 0u,
                    e >> 1 == 3 ? one : 0u};
  }
  f32x16 sacc[SCAT ? NT : 1];
  if constexpr (CVK) {
    if (mat_tile >= 0) {
#pragma unroll
      for (int i = 0; i < NT; ++i) cset(i, f32x16{});
    }
  }
#pragma unroll
  for (int i = 0; i < (SCAT ? NT : 1); ++i) sacc[i] = f32x16{};

  // The next block's K (and V^T) tile and mean are loaded into registers while this block
  // is processed, then stored into LDS at the top of the next iteration.
  constexpr int KCH = G::kTileBytes / 16 / NTHR;  // 16-byte chunks per thread per tile
  u32x4 kpre[KCH], vpre[CVK ? KCH : 1];
  float mpre = 0.0f;
  auto load_block = [&](int j) {
    const u32x4* ks = reinterpret_cast<const u32x4*>(a.kp + ((int64_t)bank * a.tb + j) * G::kTileElems);
#pragma unroll
    for (int i = 0; i < KCH; ++i) kpre[i] = ks[t + NTHR * i];
    if constexpr (CVK) {
      const u32x4* vs = reinterpret_cast<const u32x4*>(a.vp + ((int64_t)bank * a.tb + j) * G::kTileElems);
#pragma unroll
      for (int i = 0; i < KCH; ++i) vpre[i] = vs[t + NTHR * i];
    }
    if (t < D) mpre = a.kmean[((int64_t)bank * a.nb + j) * D + t];
  };
  if (j0 < j1) load_block(j0);
  for (int j = j0; j < j1; ++j) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < KCH; ++i) reinterpret_cast<u32x4*>(k_lds)[t + NTHR * i] = kpre[i];
    if constexpr (CVK) {
#pragma unroll
      for (int i = 0; i < KCH; ++i) reinterpret_cast<u32x4*>(v_lds)[t + NTHR * i] = vpre[i];
    }
    if (t < D) kmean_s[t] = mpre;
    if (j + 1 < j1) load_block(j + 1);
    const int count = min(kBlock, a.n_video - j * kBlock);
    __syncthreads();

    if constexpr (KC) {
      // Centred keys, transposed to [D][128 positions] (position p holds key swap23(p)).
      for (int cc = t; cc < D * 16; cc += NTHR) {
        const int n = cc >> 4, c = cc & 15;
        unsigned whi[4], wlo[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          float hv[2], lv[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int key = swap23(8 * c + e + u);
            float x = 0.0f;
            if (key < count) {
              const uint16_t raw = *reinterpret_cast<const uint16_t*>(
                  k_lds + G::k_off(key, n >> 3) + ((n & 7) << 1));
              x = T::to_f(raw) - kmean_s[n];
            }
            hv[u] = T::to_f(T::from_f(x));
            lv[u] = x - hv[u];
          }
          whi[e >> 1] = pack2<T>(hv[0], hv[1]);
          wlo[e >> 1] = pack2<T>(lv[0], lv[1]);
        }
        *reinterpret_cast<u32x4*>(kc_hi + G::vt_off(n, c)) = u32x4{whi[0], whi[1], whi[2], whi[3]};
        *reinterpret_cast<u32x4*>(kc_lo + G::vt_off(n, c)) = u32x4{wlo[0], wlo[1], wlo[2], wlo[3]};
      }
      __syncthreads();
    }

    if constexpr (ROT) {
      if (rot_tile >= 0) {
        f32x16 racc[4];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
          racc[tt] = f32x16{};
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            const u32x4 ka = lds_load16(k_lds, G::k_off(32 * tt + l32, 2 * s + g));
            racc[tt] = T::mfma32(ka, ub[s], racc[tt]);
          }
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            const u32x4 ka = lds_load16(k_lds, G::k_off(32 * tt + l32, 2 * s + g));
            racc[tt] = T::mfma32(ka, ub[NS + s], racc[tt]);
          }
        }
        float s1 = 0.0f;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
          for (int rr = 0; rr < 16; ++rr)
            if (32 * tt + mfma_row(rr, g) < count) s1 += racc[tt][rr];
        const float fc = (float)count;
        const float mean = pair_sum(s1) / fc;
        float s2 = 0.0f;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
          for (int rr = 0; rr < 16; ++rr)
            if (32 * tt + mfma_row(rr, g) < count) {
              const float dlt = racc[tt][rr] - mean;
              s2 += dlt * dlt;
            }
        const float var = fmaxf(pair_sum(s2) / fc, 0.0f);
        if (g == 0) a.var[((int64_t)bank * a.nb + j) * D + 32 * rot_tile + l32] = var;
      }
    }

    if constexpr (CVK) {
      if (mat_tile >= 0) {
        // C_vk[:, n] for this wave's 32 columns n.  The centred keys come from the matrix
        // core: the K rows times an identity slice, accumulated onto -kbar[n], land in the
        // output layout (lane = column n, registers = 16 tokens in swap23 order), which is
        // the B operand of V^T Kc against the V^T tile's positions -- no transpose in LDS.
        const float neg_mean = -kmean_s[32 * mat_tile + l32];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
          f32x16 kc;
#pragma unroll
          for (int r = 0; r < 16; ++r) kc[r] = neg_mean;
#pragma unroll
          for (int hh = 0; hh < 2; ++hh)
            kc = T::mfma32(lds_load16(k_lds, G::k_off(32 * tt + l32, 4 * mat_tile + 2 * hh + g)),
                           bid[hh], kc);
          if (count < kBlock) {
#pragma unroll
            for (int r = 0; r < 16; ++r)
              if (32 * tt + mfma_row(r, g) >= count) kc[r] = 0.0f;
          }
          // hi + lo pair of the centred key, as in the staged path.
          u32x4 bhi[2], blo[2];
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            unsigned whi[4], wlo[4];
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
              const float x0 = kc[8 * hh + e], x1 = kc[8 * hh + e + 1];
              const float h0 = T::to_f(T::from_f(x0)), h1 = T::to_f(T::from_f(x1));
              whi[e >> 1] = pack2<T>(h0, h1);
              wlo[e >> 1] = pack2<T>(x0 - h0, x1 - h1);
            }
            bhi[hh] = u32x4{whi[0], whi[1], whi[2], whi[3]};
            blo[hh] = u32x4{wlo[0], wlo[1], wlo[2], wlo[3]};
          }
#pragma unroll
          for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int mt = 0; mt < NT; ++mt) {
              const u32x4 va = lds_load16(v_lds, G::vt_off(32 * mt + l32, 4 * tt + 2 * hh + g));
              f32x16 c = cget(mt);
              c = T::mfma32(va, bhi[hh], c);
              cset(mt, T::mfma32(va, blo[hh], c));
            }
        }
      }
    }
    if constexpr (SCAT) {
      if (mat_tile >= 0) {
        const int nrow = 32 * mat_tile + l32;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const u32x4 ahi = lds_load16(kc_hi, G::vt_off(nrow, 2 * s + g));
          const u32x4 alo = lds_load16(kc_lo, G::vt_off(nrow, 2 * s + g));
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            const int off = G::vt_off(32 * nt + l32, 2 * s + g);
            const u32x4 bhi = lds_load16(kc_hi, off), blo = lds_load16(kc_lo, off);
            sacc[nt] = T::mfma32(ahi, bhi, sacc[nt]);
            sacc[nt] = T::mfma32(ahi, blo, sacc[nt]);
            sacc[nt] = T::mfma32(alo, bhi, sacc[nt]);
          }
        }
      }
    }
  }

  if (mat_tile >= 0) {
    const int64_t pbase = ((int64_t)bank * a.groups + grp) * D * D;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        // cacc[nt]: rows m of tile nt, this wave's columns; sacc[nt]: this wave's rows n,
        // columns of tile nt.
        if constexpr (CVK)
          a.cvk_part[pbase + (int64_t)(32 * nt + mfma_row(rr, g)) * D + 32 * mat_tile + l32] =
              cget(nt)[rr];
        if constexpr (SCAT)
          a.scat_part[pbase + (int64_t)(32 * mat_tile + mfma_row(rr, g)) * D + 32 * nt + l32] =
              sacc[nt][rr];
      }
  }
}

template <class T, int D>
static hipError_t launch_closure(const ClosureArgs& a, int flags, hipStream_t s) {
  const dim3 grid((unsigned)(a.banks * a.groups));
  switch (flags) {
    case kRot:
      hipLaunchKernelGGL((closure_kernel<T, D, kRot>), grid, dim3(closure_threads(D, kRot)), 0, s, a);
      break;
    case kCvk | kScatter:
      hipLaunchKernelGGL((closure_kernel<T, D, kCvk | kScatter>), grid,
                         dim3(closure_threads(D, kCvk | kScatter)), 0, s, a);
      break;
    case kRot | kCvk:
      hipLaunchKernelGGL((closure_kernel<T, D, kRot | kCvk>), grid,
                         dim3(closure_threads(D, kRot | kCvk)), 0, s, a);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t run_closure(const ClosureArgs& a, int dtype, int dim, int flags, hipStream_t s) {
  if (dtype == BF16::code) return dim == 128 ? launch_closure<BF16, 128>(a, flags, s) : launch_closure<BF16, 64>(a, flags, s);
  return dim == 128 ? launch_closure<F16, 128>(a, flags, s) : launch_closure<F16, 64>(a, flags, s);
}

__global__ __launch_bounds__(256) void partial_reduce_kernel(const float* part, int banks, int groups,
                                                             int elems, float divisor, float* out) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)banks * elems) return;
  const int64_t bank = idx / elems, e = idx % elems;
  const float* p = part + bank * groups * (int64_t)elems + e;
  // Sequential order of the groups (fixed, so the result does not depend on the launch);
  // unrolled so the loads of eight groups are in flight together.
  float acc = p[0];
#pragma unroll 8
  for (int i = 1; i < groups; ++i) acc += p[(int64_t)i * elems];
  out[idx] = acc / divisor;
}

hipError_t run_partial_reduce(const float* part, int banks, int groups, int elems, float divisor,
                              float* out, hipStream_t s) {
  const int64_t total = (int64_t)banks * elems;
  hipLaunchKernelGGL(partial_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                     part, banks, groups, elems, divisor, out);
  return hipGetLastError();
}

// One workgroup per padded table row (bank, j), j < ntiles * 32: fold_rank of the rotated
// variance (recap/sparse/closure.py:96-104), then w, kbar, vbar rounded to the query type
// and written as row j of their tables, plain row-major D-element rows (rows j >= nb are
// zero); the non-folded w row holds its columns in swap23 order.  FOLD writes w as the
// kFoldCols-feature row [w_0 .. w_{r-1}, rho, rho, rho, 0 ...] (natural order), 32 bytes.
template <class T, int D, bool FOLD>
__global__ __launch_bounds__(128) void tables_kernel(TablesArgs a) {
  __shared__ float red[128];
  __shared__ float vals[128];
  const int ntiles = (a.nb + kCoarseSlots - 1) / kCoarseSlots;
  const int bank = blockIdx.x / (ntiles * kCoarseSlots);
  const int j = blockIdx.x % (ntiles * kCoarseSlots);
  const bool real = j < a.nb;
  const int64_t row = (int64_t)bank * a.nb + j;
  const int t = threadIdx.x;
  const float v = (real && t < D) ? a.var[row * D + t] : 0.0f;
  const bool fold = a.rank > 0 && a.rank < D;
  red[t] = (fold && t >= a.rank && t < D) ? v : 0.0f;
  __syncthreads();
  for (int h = 64; h >= 1; h >>= 1) {
    if (t < h) red[t] += red[t + h];
    __syncthreads();
  }
  const float residual = fold ? red[0] / (float)(D - a.rank) : 0.0f;
  vals[t] = (fold && t >= a.rank) ? residual : v;
  __syncthreads();
  if (t < D) {
    // Row j of the bank's tables: element t of block j (zeros past the last block).
    const int64_t at = ((int64_t)bank * ntiles * kCoarseSlots + j) * D + t;
    a.kbar_t[at] = real ? T::from_f(a.kmean[row * D + t]) : (uint16_t)0;
    a.vbar_t[at] = real ? T::from_f(a.vmean[row * D + t]) : (uint16_t)0;
    if constexpr (FOLD) {
      if (t < kFoldCols) {
        const float f = t < a.rank ? vals[t] : (t < a.rank + 3 ? residual : 0.0f);
        a.w_t[((int64_t)bank * ntiles * kCoarseSlots + j) * kFoldCols + t] =
            real ? T::from_f(f) : (uint16_t)0;
      }
    } else {
      a.w_t[at] = real ? T::from_f(vals[swap23(t)]) : (uint16_t)0;  // columns in swap23 order
    }
  }
}

hipError_t run_tables(const TablesArgs& a, int dtype, hipStream_t s) {
  const int ntiles = (a.nb + kCoarseSlots - 1) / kCoarseSlots;
  const dim3 grid((unsigned)(a.banks * ntiles * kCoarseSlots)), block(128);
  const bool fold = coarse_folded(dtype, a.dim, a.rank);
  if (dtype == BF16::code) {
    if (a.dim == 128) {
      if (fold) hipLaunchKernelGGL((tables_kernel<BF16, 128, true>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((tables_kernel<BF16, 128, false>), grid, block, 0, s, a);
    } else {
      if (fold) hipLaunchKernelGGL((tables_kernel<BF16, 64, true>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((tables_kernel<BF16, 64, false>), grid, block, 0, s, a);
    }
  } else {
    if (a.dim == 128) hipLaunchKernelGGL((tables_kernel<F16, 128, false>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((tables_kernel<F16, 64, false>), grid, block, 0, s, a);
  }
  return hipGetLastError();
}

template <class T>
__global__ __launch_bounds__(256) void basis_tables_kernel(BasisArgs a) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int D = a.dim;
  if (idx >= (int64_t)a.banks * D * D) return;
  const int64_t bank = idx / ((int64_t)D * D);
  const int o = (int)((idx / D) % D), d = (int)(idx % D);
  const float u = a.basis[(bank * D + d) * D + o];  // U[d][o], eigenvectors in columns
  const uint16_t hi = T::from_f(u);
  if (a.u_hi_t) a.u_hi_t[idx] = hi;
  if (a.u_lo_t) a.u_lo_t[idx] = T::from_f(u - T::to_f(hi));
  if (a.u_t) a.u_t[idx] = hi;
  if (a.cvk_t) a.cvk_t[idx] = T::from_f(a.cvk[idx]);  // C_vk[m][d], row-major
}

hipError_t run_basis_tables(const BasisArgs& a, int dtype, hipStream_t s) {
  const int64_t total = (int64_t)a.banks * a.dim * a.dim;
  const dim3 grid((unsigned)((total + 255) / 256)), block(256);
  if (dtype == BF16::code) hipLaunchKernelGGL(basis_tables_kernel<BF16>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(basis_tables_kernel<F16>, grid, block, 0, s, a);
  return hipGetLastError();
}

}  // namespace recap
