// Stage 3: the corrected coarse tail over each query block's omitted key blocks.
//
// Math of recap/kernels/coarse_tail.py:79-186 with the wrapper steps of :224-312 and
// recap/sparse/attention.py:187-195, 224-230 fused in:
//   qsq   = (U^T q)^2      in the query type  (recap/sparse/closure.py:84-86)
//   drift = s C_vk q       in the query type  (recap/sparse/closure.py:89-93)
//   l_j   = s q.kbar_j + ln n_j + [s^2 qsq.w_j <= theta^2] (s^2/2) qsq.w_j
//   out   = softmax(l) . vbar  (+ g * drift, g = gated share of the mass), lse = m + ln l
// over the omitted blocks j (~partition[i, j]).  Each workgroup first compacts its
// partition row into the ascending list of its omitted blocks (a ballot count per wave and
// chunk, one scan), then walks that list in tiles of 32 blocks gathered from the tables, so
// only omitted blocks are computed and no host-side planning or synchronisation is needed
// (recap/sparse/planner.py:24-27 is the host sync this removes).
//
// One workgroup = one (bank, 128-row query block), 4 waves x 32 rows.  The contractions
// per 32-block tile (q.kbar, qsq.w, p.vbar) run on 32x32x16 MFMA with the same
// register-resident layout trick as the attention kernel: the fp32 result of one MFMA is the B operand of the next, the w table's
// columns are stored in the matching swap23 order, and vbar is read slot-major through the
// transposing LDS read.  The tile loop is pipelined: a tile's score chains run on the
// matrix cores while the previous tile's softmax runs on the VALU.  Also writes per-block
// partial sums of (gl - gl_ref) for the per-bank drift centre (recap/operator.py:148-150).
#include <array>

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
  constexpr int kScan = kMaxVideoBlocks / 256;     // chunks of the partition row
  static_assert(2 * kStage >= kMatBytes, "a staged D x D matrix spans both stages");
  static_assert(!FOLD || kWBytes == 1024, "a folded w tile is 4 bytes per thread");
  static_assert(4 * kScan <= 64, "the chunk counts are scanned by one wave");
  // Two tile stages in separate arrays, each access naming one of them at compile time: the
  // compiler can then tell that reads of one stage do not touch the copies filling the other,
  // and does not wait for those copies first.  A staged D x D matrix (U^T, C_vk) keeps rows
  // 0 .. D/2-1 in stage 0 and the rest in stage 1 (same swizzle: it depends on the row's low
  // bits only).
  __shared__ __attribute__((aligned(16))) char st0[kStage];
  __shared__ __attribute__((aligned(16))) char st1[kStage];
  // This query block's omitted blocks, ascending, then zeros up to the next multiple of 32.
  __shared__ uint16_t olist[kMaxVideoBlocks + kCoarseSlots];
  __shared__ int counts[4 * kScan + 1];
  __shared__ float wsum[4];
  __shared__ float feat[FOLD ? 4 * 32 * kFoldCols : 1];  // folded qsq features per row

  const int t = threadIdx.x, lane = t & 63, g = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lin = xcd_linear(blockIdx.x, a.banks * a.qtiles);
  const int bank = lin / a.qtiles, qt = lin % a.qtiles;
  const int b = bank / a.heads, h = bank % a.heads;
  const int ntiles = (a.nb + kCoarseSlots - 1) / kCoarseSlots;  // table rows / 32

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
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(st0 + 4096 * i + 1024 * wave), 16,
                                               from, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(st1 + 4096 * i + 1024 * wave), 16,
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
    return rt < NDT / 2 ? lds_load16(st0, G::k_off(32 * rt + l32, chunk))
                        : lds_load16(st1, G::k_off(32 * (rt - NDT / 2) + l32, chunk));
  };
  // U^T and this wave's row-map entry are requested before the partition row, so all three
  // arrive in one wait.
  stage_matrix(a.u_t + (int64_t)bank * D * D);  // U^T
  const int r = qt * kBlock + wave * 32 + l32;  // always < rows
  const int nat = a.rowmap[r];

  // The omitted blocks of this query block (partition 0), compacted in ascending order into
  // olist: block j's place is the number of omitted blocks before it, i.e. the counts of the
  // earlier (chunk of 256, wave) pairs, scanned by one wave, plus the omitted lanes below it
  // in its ballot.  All of the row's loads are issued before the first ballot, and the Q
  // row (which waits only for the row-map entry) in between.  Rows of up to 1,024 blocks
  // (every shape here) take a copy of the scan unrolled over 4 chunks instead of 16.
  u32x4 qreg[NS];
  int n_om;
  {
    const uint8_t* prow = a.partition + ((int64_t)bank * a.nb + qt) * a.nb;
    const int nchunks = (a.nb + 255) / 256;
    auto compact = [&](auto nc_tag) {
      constexpr int NC = decltype(nc_tag)::value;  // chunks unrolled (>= nchunks)
      uint8_t cell[NC];
#pragma unroll
      for (int i = 0; i < NC; ++i) cell[i] = prow[min(256 * i + t, a.nb - 1)];  // in the row
      const uint16_t* qrow = a.q + b * a.sB + h * a.sH + (int64_t)nat * a.sN;
#pragma unroll
      for (int s = 0; s < NS; ++s) qreg[s] = *reinterpret_cast<const u32x4*>(qrow + 16 * s + 8 * g);
      unsigned flags = 0;
#pragma unroll
      for (int i = 0; i < NC; ++i)
        if (256 * i + t < a.nb && cell[i] == 0) flags |= 1u << i;
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        if (i < nchunks) {  // uniform
          const unsigned long long bal = __ballot((flags >> i) & 1u);
          if (lane == 0) counts[4 * i + wave] = (int)__popcll(bal);
        }
      }
      __syncthreads();
      if (wave == 0) {  // exclusive prefix of the 4 * nchunks counts, the total after them
        const int n = 4 * nchunks;
        const int own = lane < n ? counts[lane] : 0;
        int v = own;
#pragma unroll
        for (int off = 1; off < 4 * NC; off <<= 1) {
          const int u = __shfl_up(v, off, 64);
          if (lane >= off) v += u;
        }
        if (lane < n) counts[lane] = v - own;
        if (lane == 4 * NC - 1) counts[4 * kScan] = v;
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        if (i < nchunks) {  // uniform
          const unsigned long long bal = __ballot((flags >> i) & 1u);
          if ((flags >> i) & 1u)
            olist[counts[4 * i + wave] + (int)__popcll(bal & ((1ull << lane) - 1ull))] =
                (uint16_t)(256 * i + t);
        }
      }
    };
    if (nchunks <= 4) compact(std::integral_constant<int, 4>{});
    else compact(std::integral_constant<int, kScan>{});
    n_om = __builtin_amdgcn_readfirstlane(counts[4 * kScan]);
    if (t < kCoarseSlots) olist[n_om + t] = 0;  // padding slots read table row 0
  }

  staged_barrier();

  // Tiles of 32 omitted blocks (the last one padded), gathered into LDS by buffer loads from
  // the tables (rows of the query type, one per key block): each lane copies the 16-byte
  // chunk its LDS position holds, K-tile layout with the compacted slot as the row, so kbar,
  // vbar and w images read exactly like packed tiles.  Padding slots read table row 0 and
  // are masked on the last tile.  The loop is pipelined across tiles: while the softmax and
  // p.vbar of tile i run, the q.kbar and qsq.w chains of tile i+1 run on the matrix cores,
  // so a wave's MFMAs overlap its own VALU work.  Tile i lives in stage i % 2 (layout: kbar,
  // vbar, w images); its kbar and w images arrive two tiles ahead (they are read one tile
  // ahead), its vbar image one tile ahead.
  const int ntc = (n_om + kCoarseSlots - 1) / kCoarseSlots;
  const int bank_tab = ntiles * kTabBytes;
  const int64_t tab_elems = (int64_t)bank * ntiles * kCoarseSlots * D;
  const int64_t w_elems = (int64_t)bank * ntiles * (kWBytes / 2);
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(a.kbar + tab_elems), 0, bank_tab, kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.w + w_elems), 0, ntiles * kWBytes, kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(a.vbar + tab_elems), 0, bank_tab, kBufferRsrcWord3);
  auto slot_block = [&](int c, int s) {  // table row of compacted slot s of tile c
    return (int)olist[kCoarseSlots * c + s];
  };
  // Byte offset in a D-wide table of the chunk at LDS position `pos` of a tile image.
  auto gather_src = [&](int c, int pos) {
    const int row = pos / (2 * D), pc = (pos % (2 * D)) >> 4;
    return slot_block(c, row) * 2 * D + ((pc ^ G::swz(row, NCH)) << 4);
  };
  auto copy_kw = [&](int c, char* dst) {  // kbar and w images of tile c
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      const int lo = 4096 * i + 1024 * wave, src = gather_src(c, 4096 * i + 16 * t);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void*)(dst + lo), 16, src, 0, 0, 0);
      if constexpr (!FOLD)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (lds_void*)(dst + 2 * kTabBytes + lo), 16, src, 0, 0, 0);
    }
    if constexpr (FOLD) {  // 1 KB: 4 bytes per thread, row t / 8 of 32-byte rows
      const int src = slot_block(c, t >> 3) * (kWBytes / kCoarseSlots) + 4 * (t & 7);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (lds_void*)(dst + 2 * kTabBytes + 256 * wave), 4,
                                               src, 0, 0, 0);
    }
  };
  auto copy_v = [&](int c, char* dst) {  // vbar image of tile c
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      const int lo = 4096 * i + 1024 * wave, src = gather_src(c, 4096 * i + 16 * t);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void*)(dst + kTabBytes + lo), 16, src, 0, 0, 0);
    }
  };
  // This wave's copies into LDS have landed and every wave has passed the same point.
  auto tile_barrier = [&]() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0x7 << 4);  // vmcnt(0) lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

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
    for (int rr = 0; rr < 16; rr += 2) {
      float x0 = acc[rr], x1 = acc[rr + 1];
      round2<T>(x0, x1);
      sq[rr] = x0 * x0;
      sq[rr + 1] = x1 * x1;
      if constexpr (FOLD) round2<T>(sq[rr], sq[rr + 1]);  // the full form rounds in pack2
    }
    if constexpr (FOLD) {
      // The folded form has rank <= 13 (< 16 <= mfma_row(rr >= 8, g)): only the first
      // eight registers of the first row tile can hold a leading dimension.
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const int c = 32 * ot + mfma_row(rr, g);
        if (ot == 0 && rr < 8 && c < a.rank) frow[c] = sq[rr];
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
  __syncthreads();  // the table tiles reuse the U^T staging area

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
  // Only the last tile holds padding slots (n_last of its 32 slots hold blocks) and, when
  // block nb - 1 is omitted, that short block, last in the list, at slot n_last - 1: it gets
  // its log2(n / 128) added to its q.kbar score (units of c1).
  const int n_last = n_om - kCoarseSlots * (ntc - 1);
  const bool short_omitted = n_om > 0 && olist[n_om - 1] == a.nb - 1 && short2 != 0.0f;
  const int fix_tile = n_last < kCoarseSlots || short_omitted ? ntc - 1 : -1;
  const int short_slot = short_omitted ? n_last - 1 : -1;
  const float short_add = short2 / c1;

  // The score chains of the tile in stage `st`: s = q.kbar, quad = qsq.w, each from a zero
  // accumulator.  MFMA i of the chains: folded, 0 the quad and 1 .. NS the q.kbar slices;
  // full, q.kbar slice s at 2s and qsq.w slice s at 2s+1 (each chain in slice order).
  constexpr int kScoreMfmas = FOLD ? NS + 1 : 2 * NS;
  auto score_frag = [&](const char* st, int i) {  // A operand of MFMA i
    if constexpr (FOLD) {
      return i == 0 ? lds_load16(st + 2 * kTabBytes, 32 * l32 + 16 * g)
                    : lds_load16(st, G::k_off(l32, 2 * (i - 1) + g));
    } else {
      return lds_load16(st + (i & 1 ? 2 * kTabBytes : 0), G::k_off(l32, 2 * (i >> 1) + g));
    }
  };
  auto score_mfma = [&](int i, const u32x4& f, f32x16& sacc, f32x16& wacc) {
    if constexpr (FOLD) {
      if (i == 0) wacc = T::mfma32(f, qsq_pk[0], f32x16{});
      else sacc = T::mfma32(f, qreg[i - 1], i == 1 ? f32x16{} : sacc);
    } else {
      if (i & 1) wacc = T::mfma32(f, qsq_pk[i >> 1], i == 1 ? f32x16{} : wacc);
      else sacc = T::mfma32(f, qreg[i >> 1], i == 0 ? f32x16{} : sacc);
    }
  };
  // A operand of the p.vbar MFMA (output tile dt, slot half hh): rows 32 dt + l32 (value
  // dimensions) by slots in the order of the probabilities' packing, k = 8 g + e holding
  // slot 16 hh + 8 (e / 4) + 4 g + e % 4.  The vbar image has the slots as rows, so two
  // transposing reads (ds_read_b64_tr_b16: in each group of 16 lanes, lanes 4 r .. 4 r + 3
  // supply row r of a 4 x 16 block, four 16-bit elements each, and lane i receives its
  // column i) give each lane its four consecutive slots of one dimension, twice.
  // Lane (grp = lane / 16, i = lane % 16, rq = i / 4, q = i % 4) reads row 16 hh + 8 e4 + 4 g
  // + rq at dimensions d .. d+3, d = 32 dt + 16 (grp % 2) + 4 q: chunk c = d / 8 of the row,
  // stored at c ^ swz(row).  At D = 128, swz(row) = row % 16, and bits 0-1 of c ^ swz
  // depend on the lane only, while bits 2-3 are x ^ g with x = dt ^ 2 e4 known at compile
  // time: x + g for even x, x - g for odd x.  Two per-lane bases then serve every read, the
  // rest being the instruction's immediate offset.
  const int vgrp = lane >> 4, vrq = (lane >> 2) & 3, vq = lane & 3;
  const int vlane = 256 * vrq + 16 * (((2 * (vgrp & 1) + (vq >> 1)) ^ vrq) & 3) + 8 * (vq & 1) +
                    1024 * g;
  const int vb_even = vlane + 64 * g, vb_odd = vlane - 64 * g;
  auto vbar_off = [&](int dt, int hh, int e4) {
    if constexpr (D == 128) {
      const int x = dt ^ (2 * e4);
      return (x & 1 ? vb_odd : vb_even) + 4096 * hh + 2048 * e4 + 64 * x;
    } else {
      const int row = 16 * hh + 8 * e4 + 4 * g + vrq;
      const int d = 32 * dt + 16 * (vgrp & 1) + 4 * vq;
      return row * 2 * D + (((d >> 3) ^ G::swz(row, NCH)) << 4) + 8 * ((d >> 2) & 1);
    }
  };
  auto vbar_frag = [&](const char* vt, int dt, int hh) {
    u32x4 out;
#pragma unroll
    for (int e4 = 0; e4 < 2; ++e4) {
      const u32x2 v = __builtin_bit_cast(
          u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((s16x4_lds*)(vt + vbar_off(dt, hh, e4))));
      out[2 * e4] = v[0];
      out[2 * e4 + 1] = v[1];
    }
    return out;
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

  // Lane (g, l32) holds slots mfma_row(rr, g).  The log-count ln 128 common to every full
  // block is left out of the scores and added to the LSE at the end (softmax, gated share
  // and output do not depend on it).  On the last tile, a rare branch gives the padding
  // slots s = -inf (p = exp2(-inf) = 0) and the short block its log-count.
  auto tail_fix = [&](int c, f32x16& sacc) {
    if (c == fix_tile) {
      int nl = n_last, ss = short_slot;
      asm volatile("" : "+s"(nl), "+s"(ss));  // keeps the compares in this rare branch
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const int slot = mfma_row(rr, g);
        sacc[rr] = slot >= nl ? -INFINITY : (slot == ss ? sacc[rr] + short_add : sacc[rr]);
      }
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

  // The score chains of the tile in stage `st` into sn/wn, from its first two A operands
  // (f01, read from LDS by the caller).  With a softmax to do (`probs`), the first pass of
  // the probabilities of the current tile's scores (sacc/wacc) is spread over the chain:
  // each MFMA is followed by one or two slots' probabilities, so the wave issues them while
  // the MFMA runs (the chain's MFMAs depend on each other), and the A operands are read
  // from LDS two MFMAs ahead.
  auto first_frags = [&](const char* st) {
    return std::array<u32x4, 2>{score_frag(st, 0), score_frag(st, 1)};
  };
  auto scores = [&](const char* st, const std::array<u32x4, 2>& f01, f32x16& sn, f32x16& wn,
                    auto probs, const f32x16& sacc, const f32x16& wacc, float* p, float& part,
                    float& gpart) {
    u32x4 f[3];
    f[0] = f01[0];
    f[1] = f01[1];
    part = 0.0f;
    gpart = 0.0f;
#pragma unroll
    for (int i = 0; i < kScoreMfmas; ++i) {
      if (i + 2 < kScoreMfmas) f[(i + 2) % 3] = score_frag(st, i + 2);
      score_mfma(i, f[i % 3], sn, wn);
      if constexpr (decltype(probs)::value) {
#pragma unroll
        for (int rr = 16 * i / kScoreMfmas; rr < 16 * (i + 1) / kScoreMfmas; ++rr)
          prob(rr, sacc, wacc, p, part, gpart);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // The rest of a tile after the first pass of its probabilities: the check of their sums
  // (and the redo with a raised m2), the running sums and the p.vbar product (vbar image in
  // stage `st`).
  auto finish_tile = [&](const char* st, const f32x16& sacc, const f32x16& wacc, float* p,
                         float part, float gpart) {
    const char* vt_lds = st + kTabBytes;
    if (__any(!(part <= kSumCap))) {
      // Raise m2 to the running max over this tile's slots (both lanes of a row; a padding
      // slot's score is -inf).  On the first tile, where m2 = -inf, the padding slots gave
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
      for (int hh = 0; hh < 2; ++hh) oacc[dt] = T::mfma32(vbar_frag(vt_lds, dt, hh), pk[hh], oacc[dt]);
  };

  // One step i: tile i (scores in sacc/wacc, vbar in stage `cur`) and the scores of tile
  // i+1 (kbar/w in stage `nxt`).  Copies issued: kbar/w of tile i+2 into `cur` (its kbar/w,
  // those of tile i, were read in step i-1) and vbar of tile i+1 into `nxt` (its vbar, that
  // of tile i-1, was read in step i-1).  Past the last tile the scores computed are of stale
  // LDS contents and unused.
  f32x16 sacc, wacc;
  auto step = [&](int c, char* cur, char* nxt) {
    tile_barrier();
    const std::array<u32x4, 2> f01 = first_frags(nxt);
    if (c + 2 < ntc) copy_kw(c + 2, cur);
    if (c + 1 < ntc) copy_v(c + 1, nxt);
    tail_fix(c, sacc);
    f32x16 sn, wn;
    float p[16], part, gpart;
    scores(nxt, f01, sn, wn, std::true_type{}, sacc, wacc, p, part, gpart);
    finish_tile(cur, sacc, wacc, p, part, gpart);
    sacc = sn;
    wacc = wn;
  };
  if (ntc > 0) {
    copy_kw(0, st0);
    copy_v(0, st0);
    if (ntc > 1) copy_kw(1, st1);
    tile_barrier();
    {
      float p[16], part, gpart;
      scores(st0, first_frags(st0), sacc, wacc, std::false_type{}, sacc, wacc, p, part, gpart);
    }
    for (int c = 0;; c += 2) {
      step(c, st0, st1);
      if (c + 1 >= ntc) break;
      step(c + 1, st1, st0);
      if (c + 2 >= ntc) break;
    }
  }

  // Value drift s C_vk q in the output layout: stage C_vk over the tables' LDS.
  __syncthreads();
  stage_matrix(a.cvk + (int64_t)bank * D * D);
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
      // o = (oacc / l) and gd = g * (drift) with drift = (dacc) * s, each (.) rounded to
      // the query type; two values per conversion.
      float o[4], dv[4], v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o[e] = oacc[dt][4 * q4 + e] * inv_l;
        dv[e] = dacc[4 * q4 + e];
      }
#pragma unroll
      for (int e = 0; e < 4; e += 2) {
        round2<T>(o[e], o[e + 1]);
        round2<T>(dv[e], dv[e + 1]);
        dv[e] *= a.scale;
        dv[e + 1] *= a.scale;
        round2<T>(dv[e], dv[e + 1]);
        float gd0 = gfrac * dv[e], gd1 = gfrac * dv[e + 1];
        round2<T>(gd0, gd1);
        v[e] = (has_tail ? o[e] : 0.0f) + gd0;
        v[e + 1] = (has_tail ? o[e + 1] : 0.0f) + gd1;
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
