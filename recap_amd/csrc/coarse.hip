// Stage 3: the corrected coarse tail over each query block's omitted key blocks.
//
// Math of recap/kernels/coarse_tail.py:79-186 with the wrapper steps of :224-312 and
// recap/sparse/attention.py:187-195, 224-230 fused in:
//   qsq   = (U^T q)^2      in the query type  (recap/sparse/closure.py:84-86)
//   drift = s C_vk q       in the query type  (recap/sparse/closure.py:89-93)
//   l_j   = s q.kbar_j + ln n_j + [s^2 qsq.w_j <= theta^2] (s^2/2) qsq.w_j
//   out   = softmax(l) . vbar  (+ g * drift, g = gated share of the mass), lse = m + ln l
// over the omitted blocks j (~partition[i, j]), walked in 32-block tiles of the tables with
// the partition row as a bit mask (tiles without an omitted block are skipped), so no
// host-side planning or synchronisation is needed (recap/sparse/planner.py:24-27 is the
// host sync this removes).
//
// One workgroup = one (bank, 128-row query block), 4 waves x 32 rows.  The contractions
// per 32-block tile (q.kbar, qsq.w, p.vbar, and one MFMA that puts -inf on the kept blocks'
// scores) run on 32x32x16 MFMA with the same register-resident layout trick as the
// attention kernel: the fp32 result of one MFMA is the B operand of the next, and the
// tables' columns (w) or rows (vbar^T) are stored in the matching swap23 order, as tile
// images copied verbatim into LDS.  The tile loop is pipelined: a tile's score chains run
// on the matrix cores while the previous tile's softmax runs on the VALU.  Also writes
// per-block partial sums of (gl - gl_ref) for the per-bank drift centre
// (recap/operator.py:148-150).
#include "kernels.hpp"

namespace recap {

constexpr int kMaxVideoBlocks = 4096;

template <class T, int D, bool FOLD>
__global__ __launch_bounds__(256, 2) void coarse_kernel(CoarseArgs a) {
#pragma clang fp contract(off)
  using G = TileGeom<D>;
  constexpr int NS = D / 16, NDT = D / 32, NCH = D / 8;
  constexpr int kMatBytes = D * D * 2;
  constexpr int kTabBytes = kCoarseSlots * D * 2;  // one kbar or vbar tile image
  // One w tile image: the folded features (32 rows of kFoldCols) or a full K-tile layout.
  constexpr int kWBytes = FOLD ? kCoarseSlots * kFoldCols * 2 : kTabBytes;
  constexpr int kStage = 2 * kTabBytes + kWBytes;  // kbar, vbar, w of one tile
  constexpr int NDMA = kTabBytes / 4096;           // 16-byte copies per thread per image
  static_assert(FOLD || 2 * kStage >= kMatBytes, "a staged D x D matrix spans both stages");
  static_assert(!FOLD || kWBytes == 1024, "a folded w tile is 4 bytes per thread");
  // Two tile stages in separate arrays, each access naming one of them at compile time: the
  // compiler can then tell that reads of one stage do not touch the copies filling the other,
  // and does not wait for those copies first.  A staged D x D matrix (U^T, C_vk) keeps rows
  // 0 .. D/2-1 and the rest in two halves of the same swizzled layout (it depends on the row's
  // low bits only): in the folded kernel in a buffer of its own (43.5 + 32 KB, still two
  // workgroups per CU), so the first tiles arrive while qsq runs and C_vk while the tiles
  // do; in the full one, whose stages are larger, over stages 0 and 1.
  __shared__ __attribute__((aligned(16))) char st0[kStage];
  __shared__ __attribute__((aligned(16))) char st1[kStage];
  __shared__ __attribute__((aligned(16))) char mat[FOLD ? kMatBytes : 16];
  __shared__ unsigned omit[kMaxVideoBlocks / kCoarseSlots];
  __shared__ float wsum[4];
  __shared__ float feat[FOLD ? 4 * 32 * kFoldCols : 1];  // folded qsq features per row

  const int t = threadIdx.x, lane = t & 63, g = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lin = xcd_linear(blockIdx.x, a.banks * a.qtiles);
  const int bank = lin / a.qtiles, qt = lin % a.qtiles;
  const int b = bank / a.heads, h = bank % a.heads;
  const int ntiles = (a.nb + kCoarseSlots - 1) / kCoarseSlots;

  // Stage a D x D matrix of the query type (row-major in HBM) into LDS by buffer loads into
  // LDS, all in flight at once: one wave instruction fills 1 KB of the swizzled image in lane
  // order, so each lane fetches the logical chunk that its LDS position holds (the swizzle
  // is an XOR, its own inverse).  The caller waits (vmcnt) and synchronises before reading.
  auto stage_matrix = [&](const uint16_t* src) {
    constexpr int kHalfBytes = kMatBytes / 2;  // rows 0 .. D/2-1, and the rest
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)src, 0, kMatBytes, kBufferRsrcWord3);
#pragma unroll
    for (int i = 0; i < kHalfBytes / 4096; ++i) {
      const int pos = 4096 * i + 16 * t;  // byte position in the half image
      const int row = pos / (2 * D), pc = (pos % (2 * D)) >> 4;
      const int from = row * 2 * D + ((pc ^ G::swz(row, NCH)) << 4);
      char* lo = FOLD ? mat : st0;
      char* hi = FOLD ? mat + kHalfBytes : st1;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(lo + 4096 * i + 1024 * wave), 16,
                                               from, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(hi + 4096 * i + 1024 * wave), 16,
                                               from + kHalfBytes, 0, 0, 0);
    }
  };
  // Wait for this wave's copies into LDS (and LDS accesses), then for every wave.
  auto staged_barrier = [&]() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0x7 << 4);  // vmcnt(0) lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // Fragment of row tile `rt` (32 rows) of a staged matrix; rt is a compile-time index.
  auto matrix_frag = [&](int rt, int chunk) {
    if constexpr (FOLD)
      return rt < NDT / 2 ? lds_load16(mat, G::k_off(32 * rt + l32, chunk))
                          : lds_load16(mat + kMatBytes / 2, G::k_off(32 * (rt - NDT / 2) + l32, chunk));
    else
      return rt < NDT / 2 ? lds_load16(st0, G::k_off(32 * rt + l32, chunk))
                          : lds_load16(st1, G::k_off(32 * (rt - NDT / 2) + l32, chunk));
  };
  // U^T and this wave's row-map entry are requested before the partition row, so all three
  // arrive in one wait.
  stage_matrix(a.u_t + (int64_t)bank * D * D);  // U^T
  const int r = qt * kBlock + wave * 32 + l32;  // always < rows
  const int nat = a.rowmap[r];

  // Omitted blocks of this query block (partition 0) as one bit word per table tile.  All
  // of the row's loads are issued before the first ballot, so the scan waits once, and the
  // Q row (which waits only for the row-map entry) is requested in between.
  u32x4 qreg[NS];
  {
    const uint8_t* prow = a.partition + ((int64_t)bank * a.nb + qt) * a.nb;
    constexpr int kScan = kMaxVideoBlocks / 256;
    uint8_t cell[kScan];
#pragma unroll
    for (int i = 0; i < kScan; ++i) cell[i] = prow[min(256 * i + t, a.nb - 1)];  // in the row
    const uint16_t* qrow = a.q + b * a.sB + h * a.sH + (int64_t)nat * a.sN;
#pragma unroll
    for (int s = 0; s < NS; ++s) qreg[s] = *reinterpret_cast<const u32x4*>(qrow + 16 * s + 8 * g);
    unsigned flags = 0;
#pragma unroll
    for (int i = 0; i < kScan; ++i)
      if (256 * i + t < a.nb && cell[i] == 0) flags |= 1u << i;
#pragma unroll
    for (int i = 0; i < kScan; ++i) {
      if (256 * i >= ntiles * kCoarseSlots) break;
      const unsigned long long bal = __ballot((flags >> i) & 1u);
      const int wi = (256 * i + 64 * wave) / kCoarseSlots;
      if (lane == 0 && wi < ntiles) omit[wi] = (unsigned)bal;
      if (lane == 0 && wi + 1 < ntiles) omit[wi + 1] = (unsigned)(bal >> 32);
    }
  }

  staged_barrier();

  // Table tiles (images written by the tables kernel) are copied verbatim into LDS by
  // buffer loads over this bank's images; tiles with no omitted block are skipped.  The
  // loop is pipelined across tiles: while the softmax and p.vbar of tile t_i run, the
  // q.kbar and qsq.w chains of t_{i+1} run on the matrix cores, so a wave's MFMAs overlap
  // its own VALU work.  Tile t_i lives in stage i % 2 (layout: kbar, vbar, w images); its
  // kbar and w images arrive two tiles ahead (they are read one tile ahead), its vbar image
  // one tile ahead.
  const int bank_tab = ntiles * kTabBytes;
  const int64_t tab_elems = (int64_t)bank * ntiles * kCoarseSlots * D;
  const int64_t w_elems = (int64_t)bank * ntiles * (kWBytes / 2);
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(a.kbar + tab_elems), 0, bank_tab, kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.w + w_elems), 0, ntiles * kWBytes, kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(a.vbar + tab_elems), 0, bank_tab, kBufferRsrcWord3);
  auto copy_kw = [&](int k, char* dst) {  // kbar and w images of tile k
    const int off = __builtin_amdgcn_readfirstlane(k * kTabBytes);
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      const int lo = 4096 * i + 1024 * wave, vo = 4096 * i + 16 * t;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void*)(dst + lo), 16, vo, off, 0, 0);
      if constexpr (!FOLD)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (lds_void*)(dst + 2 * kTabBytes + lo), 16, vo, off, 0, 0);
    }
    if constexpr (FOLD) {  // 1 KB: 4 bytes per thread
      const int woff = __builtin_amdgcn_readfirstlane(k * kWBytes);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (lds_void*)(dst + 2 * kTabBytes + 256 * wave), 4,
                                               4 * t, woff, 0, 0);
    }
  };
  auto copy_v = [&](int k, char* dst) {  // vbar image of tile k
    const int off = __builtin_amdgcn_readfirstlane(k * kTabBytes);
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      const int lo = 4096 * i + 1024 * wave, vo = 4096 * i + 16 * t;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void*)(dst + kTabBytes + lo), 16, vo, off, 0, 0);
    }
  };
  // This wave's copies into LDS have landed and every wave has passed the same point.
  auto tile_barrier = [&]() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0x7 << 4);  // vmcnt(0) lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // Operands of the bias MFMA that starts each tile's q.kbar accumulator: A[slot][0] = -inf
  // for a kept slot, 0 for an omitted one; B[0][row] = 1; every other element of A and B is
  // 0, so no -inf meets a 0.  The product is -inf on the kept slots and +0 on the omitted
  // ones, where the chain then runs exactly as from a zero accumulator; a kept slot stays
  // -inf through the chain and gets p = exp2(-inf) = 0 with no per-score select.
  const unsigned bias_kept = g == 0 ? pack2<T>(-INFINITY, 0.0f) : 0u;
  const u32x4 bias_ones = u32x4{g == 0 ? pack2<T>(1.0f, 0.0f) : 0u, 0u, 0u, 0u};
  // The omitted-block words in registers (lane i of ow_lo / ow_hi holds the word of tile i /
  // 64 + i) and the tiles that have one as bit masks on the scalar unit, so the walk reads
  // no LDS for its bookkeeping.
  const unsigned ow_lo = lane < ntiles ? omit[lane] : 0u;
  const unsigned ow_hi = 64 + lane < ntiles ? omit[64 + lane] : 0u;
  const unsigned long long ne_lo = __ballot(ow_lo != 0), ne_hi = __ballot(ow_hi != 0);
  auto next_tile = [&](int k) {  // the first tile after k with an omitted block, or ntiles
    ++k;
    if (k < 64) {
      const unsigned long long m = ne_lo >> k;
      if (m) return k + (int)__builtin_ctzll(m);
      k = 64;
    }
    if (k < 128) {
      const unsigned long long m = ne_hi >> (k - 64);
      if (m) return k + (int)__builtin_ctzll(m);
    }
    return ntiles;
  };
  // Omitted-block word of tile k (0 past the last tile).
  auto omit_word = [&](int k) -> unsigned {
    if (k >= ntiles) return 0u;
    return k < 64 ? (unsigned)__builtin_amdgcn_readlane((int)ow_lo, k)
                  : (unsigned)__builtin_amdgcn_readlane((int)ow_hi, k - 64);
  };

  // The first two tiles with an omitted block; the folded kernel copies their images now,
  // while the qsq MFMAs run (both stages are free: U^T is in its own buffer).
  const int k_first = next_tile(-1);
  const int k_second = k_first < ntiles ? next_tile(k_first) : ntiles;
  if constexpr (FOLD) {
    if (k_first < ntiles) {
      copy_kw(k_first, st0);
      copy_v(k_first, st0);
      if (k_second < ntiles) copy_kw(k_second, st1);
    }
  }

  // qsq = (U^T q)^2 in the query type (rotated value rounded, then its square rounded):
  // lane (g, l32) holds dims 32 ot + mfma_row(rr, g) of its row.  Full form: qsq in the
  // B-operand layout of the quadratic form (dims in swap23 order, as the w table's
  // columns).  Folded form: the kFoldCols features [qsq_0 .. qsq_{r-1}, T_hi, T_mid, T_lo,
  // 0 ...] as one B operand, gathered through LDS (lane (g, l32) holds features 8g .. 8g+7).
  constexpr int kQsqRegs = FOLD ? 1 : NDT * 2;
  u32x4 qsq_pk[kQsqRegs];
  float* frow = feat + (wave * 32 + l32) * kFoldCols;
  if constexpr (FOLD) {
#pragma unroll
    for (int e = 0; e < 8; ++e) frow[8 * g + e] = 0.0f;
    __syncthreads();
  }
  float tail = 0.0f;
#pragma unroll
  for (int ot = 0; ot < NDT; ++ot) {
    f32x16 acc = f32x16{};
#pragma unroll
    for (int s = 0; s < NS; ++s)
      acc = T::mfma32(matrix_frag(ot, 2 * s + g), qreg[s], acc);
    float sq[16];
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      const float x = T::to_f(T::from_f(acc[rr]));
      sq[rr] = T::to_f(T::from_f(x * x));
    }
    if constexpr (FOLD) {
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const int c = 32 * ot + mfma_row(rr, g);
        if (c < a.rank) frow[c] = sq[rr];
        else tail += sq[rr];
      }
    } else {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
        qsq_pk[2 * ot + hh] = u32x4{pack2<T>(sq[8 * hh], sq[8 * hh + 1]),
                                    pack2<T>(sq[8 * hh + 2], sq[8 * hh + 3]),
                                    pack2<T>(sq[8 * hh + 4], sq[8 * hh + 5]),
                                    pack2<T>(sq[8 * hh + 6], sq[8 * hh + 7])};
    }
  }
  if constexpr (FOLD) {
    // T = sum_{c>=r} qsq_c over both lanes of the row, split into three bf16 parts.
    const float total = pair_sum(tail);
    const float hi = T::to_f(T::from_f(total));
    const float mid = T::to_f(T::from_f(total - hi));
    const float lo = T::to_f(T::from_f((total - hi) - mid));
    if (g == 0) {
      frow[a.rank] = hi;
      frow[a.rank + 1] = mid;
      frow[a.rank + 2] = lo;
    }
    __syncthreads();
    const float* f8 = frow + 8 * g;
    qsq_pk[0] = u32x4{pack2<T>(f8[0], f8[1]), pack2<T>(f8[2], f8[3]), pack2<T>(f8[4], f8[5]),
                      pack2<T>(f8[6], f8[7])};
  }
  __syncthreads();  // the full kernel's table tiles reuse the U^T staging area

  const float s32 = a.scale;
  const float ssq = (float)((double)a.scale * (double)a.scale);
  const float half = (float)(0.5 * (double)a.scale * (double)a.scale);
  const float thsq = (float)((double)a.theta * (double)a.theta);
  // The gate fl(quad * s^2) <= theta^2 as one compare quad <= thq: fl(x * s^2) is monotone in
  // x, so the quads that pass form (-inf, thq], with thq within an ulp or two of
  // theta^2 / s^2 (found by stepping; exact for every scale, not only powers of two).
  float thq = thsq / ssq;
  for (int i = 0; i < 4 && thq * ssq > thsq; ++i) thq = nextafterf(thq, -INFINITY);
  for (int i = 0; i < 4 && nextafterf(thq, INFINITY) * ssq <= thsq; ++i)
    thq = nextafterf(thq, INFINITY);
  // Scores in log2 units: c1 on q.kbar, c2 on the gated qsq.w term.
  const float c1 = s32 * kLog2e, c2 = half * kLog2e;
  const float ln_full = logf((float)kBlock);
  const float short2 = (logf((float)(a.n_video - kBlock * (a.nb - 1))) - ln_full) * kLog2e;
  const int last_tile = (a.nb - 1) / kCoarseSlots;
  // Block nb - 1 sits in slot sl = mfma_row(short_reg, g) of the last tile for the lanes
  // of half g = (sl / 4) % 2; those lanes add its log2(n / 128) in units of c1.
  const int short_slot = (a.nb - 1) % kCoarseSlots;
  const int short_reg = 4 * (short_slot >> 3) + (short_slot & 3);
  const float short_lane = g == ((short_slot >> 2) & 1) ? short2 / c1 : 0.0f;

  // The score chains of the tile in stage `st`: s = q.kbar from the bias, quad = qsq.w.
  // MFMA i of the chain: 0 the bias; folded, 1 the quad and 2 .. NS+1 the q.kbar slices;
  // full, q.kbar slice s at 2s+1 and qsq.w slice s at 2s+2 (each chain in slice order).
  constexpr int kScoreMfmas = FOLD ? NS + 2 : 2 * NS + 1;
  auto score_frag = [&](const char* st, int i) {  // A operand of MFMA i >= 1
    if constexpr (FOLD) {
      return i == 1 ? lds_load16(st + 2 * kTabBytes, 32 * l32 + 16 * g)
                    : lds_load16(st, G::k_off(l32, 2 * (i - 2) + g));
    } else {
      return lds_load16(st + ((i - 1) & 1 ? 2 * kTabBytes : 0), G::k_off(l32, 2 * ((i - 1) >> 1) + g));
    }
  };
  auto score_mfma = [&](int i, const u32x4& f, const u32x4& bias_a, f32x16& sacc, f32x16& wacc) {
    if (i == 0) {
      sacc = T::mfma32(bias_a, bias_ones, f32x16{});
    } else if constexpr (FOLD) {
      if (i == 1) wacc = T::mfma32(f, qsq_pk[0], wacc);
      else sacc = T::mfma32(f, qreg[i - 2], sacc);
    } else {
      if ((i - 1) & 1) wacc = T::mfma32(f, qsq_pk[(i - 1) >> 1], wacc);
      else sacc = T::mfma32(f, qreg[(i - 1) >> 1], sacc);
    }
  };

  // Running max m2 (log2 units), raised lazily: a tile's probabilities are first taken
  // against the current m2, and only when a lane's sum of them exceeds kSumCap (or is not
  // finite, as on the first tile where m2 = -inf) is m2 raised to the true running max and
  // the tile redone.  Every accepted probability is then <= kSumCap, exact to the type's
  // precision in fp32 and bf16, and no per-score max is taken on the common path.
  constexpr float kSumCap = 4096.0f;
  float m2 = -INFINITY, lsum = 0.0f, gsum = 0.0f;
  f32x16 oacc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) oacc[dt] = f32x16{};

  // Lane (g, l32) holds slots mfma_row(rr, g); kept slots hold s = -inf.  The log-count
  // ln 128 common to every full block is left out of the scores and added to the LSE at the
  // end (softmax, gated share and output do not depend on it); the short last block gets
  // its log2(n / 128) added to its q.kbar score (units of c1).
  auto short_fix = [&](int k, f32x16& sacc) {
    if (k == last_tile && short2 != 0.0f) {
      int sreg = short_reg;
      asm volatile("" : "+s"(sreg));  // keeps the 16 compares in this rare branch
#pragma unroll
      for (int rr = 0; rr < 16; ++rr)
        if (rr == sreg) sacc[rr] += short_lane;
    }
  };
  // Probability of slot register rr against m2: score - m2 = c1 s + (gate ? c2 quad : 0) - m2,
  // the gate term and -m2 folded into one select; part and gpart accumulate in rr order.
  auto prob = [&](int rr, const f32x16& sacc, const f32x16& wacc, float* p, float& part,
                  float& gpart) {
    const bool gate = wacc[rr] <= thq;
    const float tm = gate ? fmaf(wacc[rr], c2, -m2) : -m2;
    p[rr] = __builtin_amdgcn_exp2f(fmaf(sacc[rr], c1, tm));
    part += p[rr];
    gpart += gate ? p[rr] : 0.0f;
  };

  // The score chains of the tile in stage `st` (omitted word ow) into sn/wn.  With a
  // softmax to do (`probs`), the first pass of the probabilities of the current tile's
  // scores (sacc/wacc) is spread over the chain: each MFMA is followed by one or two slots'
  // probabilities, so the wave issues them while the MFMA runs (the chain's MFMAs depend
  // on each other), and the A operands are read from LDS two MFMAs ahead.
  auto scores = [&](const char* st, unsigned ow, f32x16& sn, f32x16& wn, auto probs,
                    const f32x16& sacc, const f32x16& wacc, float* p, float& part,
                    float& gpart) {
    // Lane (g, l32) holds A[slot l32][8g .. 8g+7] of the bias MFMA.
    const u32x4 bias_a = u32x4{(ow >> l32) & 1u ? 0u : bias_kept, 0u, 0u, 0u};
    u32x4 f[3];
    f[1] = score_frag(st, 1);
    f[2] = score_frag(st, 2);
    wn = f32x16{};
    part = 0.0f;
    gpart = 0.0f;
#pragma unroll
    for (int i = 0; i < kScoreMfmas; ++i) {
      if (i >= 1 && i + 2 < kScoreMfmas) f[(i + 2) % 3] = score_frag(st, i + 2);
      score_mfma(i, f[i % 3], bias_a, sn, wn);
      if constexpr (decltype(probs)::value) {
#pragma unroll
        for (int rr = 16 * i / kScoreMfmas; rr < 16 * (i + 1) / kScoreMfmas; ++rr)
          prob(rr, sacc, wacc, p, part, gpart);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // The rest of tile k after the first pass of its probabilities: the check of their sums
  // (and the redo with a raised m2), the running sums and the p.vbar product (vbar image in
  // stage `st`).
  auto finish_tile = [&](const char* st, const f32x16& sacc, const f32x16& wacc, float* p,
                         float part, float gpart) {
    const char* vt_lds = st + kTabBytes;
    if (__any(!(part <= kSumCap))) {
      // Raise m2 to the running max over this tile's omitted slots (both lanes of a row; a
      // kept slot's score is -inf).  On the first tile, where m2 = -inf, the kept slots gave
      // p = NaN (-inf + inf) above, which also lands here.
      float mx = -INFINITY;
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const float sc = fmaf(sacc[rr], c1, wacc[rr] <= thq ? wacc[rr] * c2 : 0.0f);
        mx = __builtin_elementwise_maximum(mx, sc);
      }
      mx = pair_max(mx);
      if (mx > m2) {
        const float alpha = __builtin_amdgcn_exp2f(m2 - mx);
        lsum *= alpha;
        gsum *= alpha;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) oacc[dt] *= alpha;
        m2 = mx;
      }
      part = 0.0f;
      gpart = 0.0f;
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) prob(rr, sacc, wacc, p, part, gpart);
    }
    lsum += part;
    gsum += gpart;
    u32x4 pk[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
      pk[hh] = u32x4{pack2<T>(p[8 * hh], p[8 * hh + 1]), pack2<T>(p[8 * hh + 2], p[8 * hh + 3]),
                     pack2<T>(p[8 * hh + 4], p[8 * hh + 5]), pack2<T>(p[8 * hh + 6], p[8 * hh + 7])};
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
        oacc[dt] = T::mfma32(lds_load16(vt_lds, coarse_vt_off(32 * dt + l32, 8 * (2 * hh + g))),
                             pk[hh], oacc[dt]);
  };

  // One step i: tile k = t_i (scores in sacc/wacc, vbar in stage `cur`) and the scores of
  // kn = t_{i+1} (kbar/w in stage `nxt`).  Copies issued: kbar/w of t_{i+2} into `cur`
  // (its kbar/w, those of t_i, were read in step i-1) and vbar of t_{i+1} into `nxt` (its
  // vbar, that of t_{i-1}, was read in step i-1).  Past the last tile the scores computed
  // are of stale LDS contents and unused.  Returns t_{i+2}.
  f32x16 sacc, wacc;
  // The folded kernel requests C_vk in the first step, after its barrier (every wave is done
  // with U^T), so the copy lands by the next one.
  bool cvk_staged = false;
  auto step = [&](int k, int kn, char* cur, char* nxt) {
    tile_barrier();
    const int kn2 = kn < ntiles ? next_tile(kn) : ntiles;
    if (kn2 < ntiles) copy_kw(kn2, cur);
    if (kn < ntiles) copy_v(kn, nxt);
    if constexpr (FOLD) {
      if (!cvk_staged) {
        stage_matrix(a.cvk + (int64_t)bank * D * D);
        cvk_staged = true;
      }
    }
    short_fix(k, sacc);
    f32x16 sn, wn;
    float p[16], part, gpart;
    scores(nxt, omit_word(kn), sn, wn, std::true_type{}, sacc, wacc, p, part, gpart);
    finish_tile(cur, sacc, wacc, p, part, gpart);
    sacc = sn;
    wacc = wn;
    return kn2;
  };
  int k = k_first;
  if (k < ntiles) {
    int kn = k_second;
    if constexpr (!FOLD) {
      copy_kw(k, st0);
      copy_v(k, st0);
      if (kn < ntiles) copy_kw(kn, st1);
    }
    tile_barrier();
    {
      float p[16], part, gpart;
      scores(st0, omit_word(k), sacc, wacc, std::false_type{}, sacc, wacc, p, part, gpart);
    }
    while (true) {
      int kn2 = step(k, kn, st0, st1);
      if (kn >= ntiles) break;
      k = kn;
      kn = kn2;
      kn2 = step(k, kn, st1, st0);
      if (kn >= ntiles) break;
      k = kn;
      kn = kn2;
    }
  }

  // Value drift s C_vk q in the output layout: C_vk in its buffer (folded; staged here only
  // when there was no tile) or staged over the tables' LDS.
  if constexpr (FOLD) {
    if (!cvk_staged) stage_matrix(a.cvk + (int64_t)bank * D * D);
  } else {
    __syncthreads();
    stage_matrix(a.cvk + (int64_t)bank * D * D);
  }
  staged_barrier();

  const float l = pair_sum(lsum);
  const float gs = pair_sum(gsum);
  const bool has_tail = l > 0.0f;
  const float safe_l = fmaxf(l, 1.0e-30f);
  const float inv_l = 1.0f / safe_l;  // one division per row instead of one per element
  const float gfrac = T::to_f(T::from_f(has_tail ? gs / safe_l : 0.0f));
  const int64_t ri = (int64_t)bank * a.rows + r;
  uint16_t* gorow = a.go + ri * D;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    f32x16 dacc = f32x16{};
#pragma unroll
    for (int s = 0; s < NS; ++s)
      dacc = T::mfma32(matrix_frag(dt, 2 * s + g), qreg[s], dacc);
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float o = has_tail ? T::to_f(T::from_f(oacc[dt][4 * q4 + e] * inv_l)) : 0.0f;
        const float dv = T::to_f(T::from_f(T::to_f(T::from_f(dacc[4 * q4 + e])) * a.scale));
        const float gd = T::to_f(T::from_f(gfrac * dv));
        v[e] = o + gd;
      }
      *reinterpret_cast<u32x2*>(gorow + 32 * dt + 8 * q4 + 4 * g) =
          u32x2{pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3])};
    }
  }
  const float lse = has_tail ? (m2 * kLn2 + logf(l)) + ln_full : -INFINITY;
  if (g == 0) a.gl[ri] = lse;
  if (a.glref != nullptr) {
    const float diff = half_wave_sum(lse - a.glref[ri]);
    if (lane == 0) wsum[wave] = diff;
    __syncthreads();
    if (t == 0) a.drift_part[(int64_t)bank * a.qtiles + qt] = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
  }
}

template <class T, int D, bool FOLD>
static hipError_t launch_coarse(const CoarseArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((coarse_kernel<T, D, FOLD>), dim3((unsigned)(a.banks * a.qtiles)), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t run_coarse(const CoarseArgs& a, int dtype, int dim, hipStream_t s) {
  if (coarse_folded(dtype, dim, a.rank))
    return dim == 128 ? launch_coarse<BF16, 128, true>(a, s) : launch_coarse<BF16, 64, true>(a, s);
  if (dtype == BF16::code)
    return dim == 128 ? launch_coarse<BF16, 128, false>(a, s) : launch_coarse<BF16, 64, false>(a, s);
  return dim == 128 ? launch_coarse<F16, 128, false>(a, s) : launch_coarse<F16, 64, false>(a, s);
}

// Per-bank drift centre c = sum(partials) / rows (recap/operator.py:148-150).
__global__ __launch_bounds__(256) void drift_center_kernel(const float* part, int tiles, int rows,
                                                           float* center) {
  __shared__ float red[256];
  const int bank = blockIdx.x, t = threadIdx.x;
  const float* p = part + (int64_t)bank * tiles;
  const int per = (tiles + 255) / 256;
  float acc = 0.0f;
  for (int i = t * per; i < min((t + 1) * per, tiles); ++i) acc += p[i];
  red[t] = acc;
  __syncthreads();
  for (int h = 128; h >= 1; h >>= 1) {
    if (t < h) red[t] += red[t + h];
    __syncthreads();
  }
  if (t == 0) center[bank] = red[0] / (float)rows;
}

hipError_t run_drift_center(const float* part, int banks, int tiles, int rows, float* center,
                            hipStream_t s) {
  hipLaunchKernelGGL(drift_center_kernel, dim3((unsigned)banks), dim3(256), 0, s, part, tiles, rows, center);
  return hipGetLastError();
}

}  // namespace recap
