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
  constexpr int NSLOT = SCAT ? 2 : 4;  // 64-key halves of the K / V^T tiles in LDS
  constexpr int KH = G::kHalfBytes, VH = CVK ? G::kHalfBytes : 16;
  __shared__ __attribute__((aligned(16))) char k_s0[KH], k_s1[KH];
  __shared__ __attribute__((aligned(16))) char k_s2[NSLOT > 2 ? KH : 16], k_s3[NSLOT > 2 ? KH : 16];
  __shared__ __attribute__((aligned(16))) char v_s0[VH], v_s1[VH];
  __shared__ __attribute__((aligned(16))) char v_s2[NSLOT > 2 ? VH : 16], v_s3[NSLOT > 2 ? VH : 16];
  __shared__ __attribute__((aligned(16))) char kc_hi[KC ? D * 256 : 16];
  __shared__ __attribute__((aligned(16))) char kc_lo[KC ? D * 256 : 16];
  __shared__ __attribute__((aligned(16))) float kmean_s[2][D];  // 16-byte copies land here

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

  // The K and V^T tiles stream through NSLOT slots of one 64-key half each (a half of
  // either image is contiguous), copied straight into LDS by buffer loads, so NSLOT - 1
  // halves are in flight while one is processed.  Each slot is an array of its own, so the
  // compiler can tell that a half's LDS reads miss the copies in flight.  The statistics
  // are taken per half in the order of the whole-block computation (tiles tt = 2 hf and
  // 2 hf + 1 of half hf, the rotated moments reduced after the second half), so the results
  // do not depend on the split.  A block's key mean is copied the same way, one block ahead,
  // into one of two LDS rows (block parity).
  constexpr int HCH = G::kHalfBytes / 16 / NTHR;  // 16-byte copies per thread per image half
  constexpr int NDMA = HCH * (CVK ? 2 : 1);        // copies per thread per half
  constexpr bool MEAN = CVK || SCAT;
  const int nh = 2 * max(j1 - j0, 0);
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.kp + (int64_t)bank * a.tb * G::kTileElems), 0, a.tb * G::kTileBytes,
      kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.vp + (int64_t)bank * a.tb * G::kTileElems), 0, CVK ? a.tb * G::kTileBytes : 0,
      kBufferRsrcWord3);
  auto slot_k = [&](auto u) -> char* {
    constexpr int U = decltype(u)::value % NSLOT;
    if constexpr (U == 0) return k_s0;
    else if constexpr (U == 1) return k_s1;
    else if constexpr (U == 2) return k_s2;
    else return k_s3;
  };
  auto slot_v = [&](auto u) -> char* {
    constexpr int U = decltype(u)::value % NSLOT;
    if constexpr (U == 0) return v_s0;
    else if constexpr (U == 1) return v_s1;
    else if constexpr (U == 2) return v_s2;
    else return v_s3;
  };
  auto copy_half = [&](int h, char* kdst, char* vdst) {
    const int src = (j0 + (h >> 1)) * G::kTileBytes + (h & 1) * G::kHalfBytes;
#pragma unroll
    for (int i = 0; i < HCH; ++i) {
      const int lo = 16 * (NTHR * i + 64 * wave), off = src + 16 * (NTHR * i + t);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void*)(kdst + lo), 16, off, 0, 0, 0);
      if constexpr (CVK)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void*)(vdst + lo), 16, off, 0, 0, 0);
    }
  };
  // This wave's copies but its last N have landed and its LDS writes are done; then every
  // wave has passed the same point.  Copies land in order, and any other vector memory
  // access counted after them only makes the wait longer.
  auto vm_barrier = [&](auto n_tag) {
    constexpr int N = decltype(n_tag)::value;
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4));  // vmcnt(N) lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  auto lds_barrier = [&]() {  // LDS writes of every wave done, copies left in flight
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (0x7 << 4));  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  const __amdgpu_buffer_rsrc_t mrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.kmean + (int64_t)bank * a.nb * D), 0, MEAN ? a.nb * D * 4 : 0, kBufferRsrcWord3);
  auto copy_mean = [&](int j) {  // wave 0, 16 bytes per lane
    if (t < D / 4)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(mrs, (lds_void*)kmean_s[(j - j0) & 1], 16,
                                               4 * j * D + 16 * t, 0, 0, 0);
  };
  if (nh > 0) {
    if constexpr (MEAN) copy_mean(j0);
    copy_half(0, k_s0, v_s0);
    copy_half(1, k_s1, v_s1);
    if constexpr (NSLOT == 4)
      if (nh > 2) copy_half(2, k_s2, v_s2);
  }

  // Half h of the group, in slot U % NSLOT (hf = U % 2 is h % 2: NSLOT is even and every
  // pass of the loop starts at a multiple of NSLOT): the copies and barriers every wave takes
  // part in, then this wave's `work`.
  auto half = [&](auto u, int h, auto& work) {
    constexpr int U = decltype(u)::value, HF = U & 1;
    const char* ks = slot_k(u);
    const char* vs = slot_v(u);
    const int jb = h >> 1, j = j0 + jb;
    // Wait for half h: the copies issued after its own are those of halves h + 1 ..
    // min(h + NSLOT - 2, nh - 1), plus at most one block mean, which only lengthens the wait.
    // A block's mean is issued before the copy of its second half, so the wait for its first
    // half, which leaves only copies of later halves outstanding, covers it.
    const int ahead = min(NSLOT - 2, nh - 1 - h);
    if (NSLOT == 4 && ahead >= 2) vm_barrier(std::integral_constant<int, 2 * NDMA>{});
    else if (NSLOT == 4 && ahead == 1) vm_barrier(std::integral_constant<int, NDMA>{});
    else vm_barrier(std::integral_constant<int, 0>{});
    if constexpr (MEAN)
      if (HF == 0 && j + 1 < j1) copy_mean(j + 1);
    // The slot of half h + NSLOT - 1 held half h - 1, which every wave has finished.
    if (h + NSLOT - 1 < nh)
      copy_half(h + NSLOT - 1, slot_k(std::integral_constant<int, U + NSLOT - 1>{}),
                slot_v(std::integral_constant<int, U + NSLOT - 1>{}));
    // Valid tokens of the block (kBlock except for a ragged last block), made scalar so that
    // the masks below are branches taken by that block only.
    const int count = __builtin_amdgcn_readfirstlane(min(kBlock, a.n_video - j * kBlock));
    const float* kmean_b = kmean_s[jb & 1];

    if constexpr (KC) {
      // Centred keys, transposed to [D][128 positions] (position p holds key swap23(p), in
      // the same half as p): positions 64 hf .. 64 hf + 63 here.
      for (int cc = t; cc < D * 8; cc += NTHR) {
        const int n = cc >> 3, c = 8 * HF + (cc & 7);
        unsigned whi[4], wlo[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          float hv[2], lv[2];
#pragma unroll
          for (int w = 0; w < 2; ++w) {
            const int key = swap23(8 * c + e + w);
            float x = 0.0f;
            if (key < count) {
              const uint16_t raw = *reinterpret_cast<const uint16_t*>(
                  ks + G::k_off(key - 64 * HF, n >> 3) + ((n & 7) << 1));
              x = T::to_f(raw) - kmean_b[n];
            }
            hv[w] = T::to_f(T::from_f(x));
            lv[w] = x - hv[w];
          }
          whi[e >> 1] = pack2<T>(hv[0], hv[1]);
          wlo[e >> 1] = pack2<T>(lv[0], lv[1]);
        }
        *reinterpret_cast<u32x4*>(kc_hi + G::vt_off(n, c)) = u32x4{whi[0], whi[1], whi[2], whi[3]};
        *reinterpret_cast<u32x4*>(kc_lo + G::vt_off(n, c)) = u32x4{wlo[0], wlo[1], wlo[2], wlo[3]};
      }
      lds_barrier();
    }
    work(u, ks, vs, j, count, kmean_b);
  };

  // A wave has one job (rot_tile or mat_tile) for the whole group, and each job runs its own
  // copy of the loop, so the registers one job keeps from half to half (the rotated tiles of
  // the block, or the C_vk accumulators) are not held through the other job's code.
  f32x16 racc[ROT ? 4 : 1];
  auto rot_work = [&](auto u, const char* ks, const char*, int j, int count, const float*) {
    constexpr int HF = decltype(u)::value & 1;
    if constexpr (ROT) {
      {
        // The half's K fragments are all requested before the first MFMA (the fence keeps
        // the compiler from moving each read next to its use, where the MFMA would wait out
        // the LDS latency); each serves the hi and the lo product.
        u32x4 ka[2][NS];
#pragma unroll
        for (int w = 0; w < 2; ++w)
#pragma unroll
          for (int s = 0; s < NS; ++s) ka[w][s] = lds_load16(ks, G::k_off(32 * w + l32, 2 * s + g));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int w = 0; w < 2; ++w) {
          const int tt = 2 * HF + w;
          racc[tt] = f32x16{};
#pragma unroll
          for (int s = 0; s < NS; ++s) racc[tt] = T::mfma32(ka[w][s], ub[s], racc[tt]);
#pragma unroll
          for (int s = 0; s < NS; ++s) racc[tt] = T::mfma32(ka[w][s], ub[NS + s], racc[tt]);
        }
        if constexpr (HF == 1) {
          // Mean, then mean squared deviation, over the block's valid tokens in token-tile
          // order; a full block (every block but a ragged last one) needs no mask.
          auto moments = [&](auto full_tag) {
            constexpr bool FULL = decltype(full_tag)::value;
            float s1 = 0.0f;
#pragma unroll
            for (int tt = 0; tt < 4; ++tt)
#pragma unroll
              for (int rr = 0; rr < 16; ++rr)
                if (FULL || 32 * tt + mfma_row(rr, g) < count) s1 += racc[tt][rr];
            const float fc = (float)count;
            const float mean = pair_sum(s1) / fc;
            float s2 = 0.0f;
#pragma unroll
            for (int tt = 0; tt < 4; ++tt)
#pragma unroll
              for (int rr = 0; rr < 16; ++rr)
                if (FULL || 32 * tt + mfma_row(rr, g) < count) {
                  const float dlt = racc[tt][rr] - mean;
                  s2 = fmaf(dlt, dlt, s2);  // explicit: a contraction could fuse either product
                }
            return fmaxf(pair_sum(s2) / fc, 0.0f);
          };
          const float var = count == kBlock ? moments(std::true_type{}) : moments(std::false_type{});
          if (g == 0) a.var[((int64_t)bank * a.nb + j) * D + 32 * rot_tile + l32] = var;
        }
      }
    }
  };
  auto mat_work = [&](auto u, const char* ks, const char* vs, int, int count,
                      const float* kmean_b) {
    constexpr int HF = decltype(u)::value & 1;
    if constexpr (CVK) {
      {
        // C_vk[:, n] for this wave's 32 columns n.  The centred keys come from the matrix
        // core: the K rows times an identity slice, accumulated onto -kbar[n], land in the
        // output layout (lane = column n, registers = 16 tokens in swap23 order), which is
        // the B operand of V^T Kc against the V^T tile's positions -- no transpose in LDS.
        const float neg_mean = -kmean_b[32 * mat_tile + l32];
#pragma unroll
        for (int w = 0; w < 2; ++w) {
          const int tt = 2 * HF + w;
          // The token tile's K and V^T fragments, all requested before its first MFMA (the
          // fence keeps them there; V^T positions 32 tt + 16 hh .. of this half are chunk
          // 4 w + 2 hh + g of its image).
          u32x4 kf[2], va[2][NT];
#pragma unroll
          for (int hh = 0; hh < 2; ++hh)
            kf[hh] = lds_load16(ks, G::k_off(32 * w + l32, 4 * mat_tile + 2 * hh + g));
#pragma unroll
          for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int mt = 0; mt < NT; ++mt)
              va[hh][mt] = lds_load16(vs, G::vt_off(32 * mt + l32, 4 * w + 2 * hh + g));
          __builtin_amdgcn_sched_barrier(0);
          f32x16 kc;
#pragma unroll
          for (int r = 0; r < 16; ++r) kc[r] = neg_mean;
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) kc = T::mfma32(kf[hh], bid[hh], kc);
          if (count < kBlock) {
#pragma unroll
            for (int r = 0; r < 16; ++r)
              if (32 * tt + mfma_row(r, g) >= count) kc[r] = 0.0f;
          }
          // hi + lo pair of the centred key, as in the staged path: the hi pair is the packed
          // rounding itself, widened back to form the lo pair.
          u32x4 bhi[2], blo[2];
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            unsigned whi[4], wlo[4];
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
              const float x0 = kc[8 * hh + e], x1 = kc[8 * hh + e + 1];
              float h0 = x0, h1 = x1;
              round2<T>(h0, h1);
              whi[e >> 1] = pack2<T>(x0, x1);
              wlo[e >> 1] = pack2<T>(x0 - h0, x1 - h1);
            }
            bhi[hh] = u32x4{whi[0], whi[1], whi[2], whi[3]};
            blo[hh] = u32x4{wlo[0], wlo[1], wlo[2], wlo[3]};
          }
#pragma unroll
          for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int mt = 0; mt < NT; ++mt) {
              f32x16 c = cget(mt);
              c = T::mfma32(va[hh][mt], bhi[hh], c);
              cset(mt, T::mfma32(va[hh][mt], blo[hh], c));
            }
        }
      }
    }
    if constexpr (SCAT) {
      {
        const int nrow = 32 * mat_tile + l32;
#pragma unroll
        for (int s = 4 * HF; s < 4 * HF + 4; ++s) {
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
  };
  auto idle = [&](auto, const char*, const char*, int, int, const float*) {};
  auto run = [&](auto work) {
    for (int h0 = 0; h0 < nh; h0 += NSLOT) {
      half(std::integral_constant<int, 0>{}, h0, work);
      half(std::integral_constant<int, 1>{}, h0 + 1, work);
      if constexpr (NSLOT == 4) {
        if (h0 + 2 >= nh) break;
        half(std::integral_constant<int, 2>{}, h0 + 2, work);
        half(std::integral_constant<int, 3>{}, h0 + 3, work);
      }
    }
  };
  if (ROT && rot_tile >= 0) run(rot_work);
  else if ((CVK || SCAT) && mat_tile >= 0) run(mat_work);
  else run(idle);

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
