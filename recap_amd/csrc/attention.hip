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
//   head   (oh, lh) in reordered order, oh rounded to the query type as the external
//          kernel's bf16 output is -- the head branch a refresh capture needs;
//   dense  output + LSE in native order -- a refresh's dense call;
//   dense-head  both of a refresh in one pass: the kept blocks are walked first, the head
//          branch is stored when they are done, then the remaining blocks complete the
//          dense output;
//   merge  head (+) [coarse tail + drift-weighted refinement] in LSE space for rows < R,
//          the head alone above (recap/kernels/detail_cache.py:220-301), written in
//          native order: the whole corrected sparse output in one pass.  The head enters
//          the merge rounded to the query type, as the reference's head tensor does.
// The masked modes walk their kept blocks in one order (a kept ragged last block first,
// then ascending), and dense-head stores its head branch before the first block after the
// kept ones can move the running max, so the head branch of head, dense-head and merge
// modes is the same bit for bit.
#include <type_traits>

#include "kernels.hpp"

namespace recap {

constexpr int kMaxTiles = 2048;

// Rows whose running max grows by less than this (log2 units) keep their stale max: p then
// stays below 2^8, exact in fp32 and bf16, and the O rescale is skipped.
constexpr float kRescaleSlack = 8.0f;

// At d = 64 a step has half the MFMA work of d = 128 for the same softmax work per score,
// so the VALU bounds it.  There the running max is instead raised only when a sub-tile's
// probabilities, taken against the current max, sum to more than kSumCap in some lane (or
// are not finite): the sub-tile is then redone against its own max, and no row max is taken
// on the common path (every accepted p is <= kSumCap, exact in fp32 and bf16).
constexpr float kSumCap = 4096.0f;

// s_waitcnt immediate (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
// that waits for all vector memory operations of this wave -- the tile copies into LDS --
// and all its LDS reads.
constexpr int kWaitVmLgkm0 = 0x7 << 4;

// Wait for this wave's copies into LDS and its LDS reads, then for every wave of the
// workgroup: afterwards the copied sub-tiles are visible and the slots read so far may be
// overwritten.  The copies count on vmcnt only, so the wait is spelled out.
__device__ inline void tile_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(kWaitVmLgkm0);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Each wave owns kGroups groups of 32 query rows, so every K/V fragment it reads from LDS
// feeds kGroups MFMAs; a 128-row query block then takes kThreads threads.  kGroups = 2
// halves the LDS reads and is correct, but at d = 128 it needs one wave per SIMD and the
// compiler then keeps every MFMA result in AGPRs: it measured slower.
constexpr int kGroups = 1;
constexpr int kRowsPerWave = 32 * kGroups;
constexpr int kThreads = 64 * (kBlock / kRowsPerWave);

// Final normalisation and store of one query row per lane pair (lane l holds output columns
// 32 dt + 8 q4 + 4 g .. +3 of the row), in the layout of the kernel's mode.
template <class T, int D, int MODE>
__device__ inline void store_rows(const AttnArgs& a, int bank, int b, int h, int r, int nat,
                                  int g, const f32x16 (&oacc)[D / 32], float m, float lt) {
  constexpr int NDT = D / 32;
  const float inv = 1.0f / lt;
  const float lse = (m + log2f(lt)) * kLn2;

  if constexpr (MODE == kModeHead) {
    // Head branch in the query type (the reference's head is the bf16 tensor its attention
    // kernel returns, recap/operator.py:366-370); the capture reads it back from here.
    uint16_t* orow = a.head_out + ((int64_t)bank * a.n_tokens + r) * D;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d0 = 32 * dt + 8 * q4 + 4 * g;
        u32x2 v = {pack2<T>(oacc[dt][4 * q4] * inv, oacc[dt][4 * q4 + 1] * inv),
                   pack2<T>(oacc[dt][4 * q4 + 2] * inv, oacc[dt][4 * q4 + 3] * inv)};
        *reinterpret_cast<u32x2*>(orow + d0) = v;
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
  // tail.  The head is rounded to the query type first: the reference merges the head
  // tensor its attention kernel stored in that type (recap/operator.py:500-509, loaded with
  // .to(float32) at recap/kernels/detail_cache.py:228-234).
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
    // One reciprocal per denominator and row instead of a division per element.
    const float rden = 1.0f / den, rden2 = 1.0f / den2;
    const uint16_t* gorow = a.go + ri * D;
    const uint16_t* drow = a.det + ri * D;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d0 = 32 * dt + 8 * q4 + 4 * g;
        const u32x2 gw = *reinterpret_cast<const u32x2*>(gorow + d0);
        const u32x2 dw = *reinterpret_cast<const u32x2*>(drow + d0);
        const u32x2 hw = {pack2<T>(oacc[dt][4 * q4] * inv, oacc[dt][4 * q4 + 1] * inv),
                          pack2<T>(oacc[dt][4 * q4 + 2] * inv, oacc[dt][4 * q4 + 3] * inv)};
        float res[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const unsigned gword = gw[e >> 1], dword = dw[e >> 1], hword = hw[e >> 1];
          const float gov = T::to_f((uint16_t)((e & 1) ? gword >> 16 : gword & 0xffff));
          const float detv = f16_to_f((uint16_t)((e & 1) ? dword >> 16 : dword & 0xffff));
          const float ohv = T::to_f((uint16_t)((e & 1) ? hword >> 16 : hword & 0xffff));
          const float to = (gov * sm + (gov + detv) * cm) * rden;
          res[e] = (ohv * wh + to * wt) * rden2;
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


template <class T, int D, int MODE>
__global__ __launch_bounds__(kThreads, 2) void attention_kernel(AttnArgs a) {
  using G = TileGeom<D>;
  constexpr int NS = D / 16;                  // k-steps over the head dimension
  constexpr int NDT = D / 32;                 // 32-row tiles of O^T
  constexpr int HALF = G::kHalfBytes;         // K or V^T image of a 64-key sub-tile
  constexpr int NDMA = HALF / (16 * kThreads);  // 16-byte copies per thread per image
  // LDS: K images of sub-tiles 2k / 2k+1 in k_lds0 / k_lds1, V^T images likewise.  Four
  // separate arrays, each access naming one of them at compile time (the step parity is
  // static): the compiler can then tell that a step's fragment reads do not touch the slots
  // its copies are filling, and does not wait for those copies before the reads.
  __shared__ __attribute__((aligned(16))) char k_lds0[HALF];
  __shared__ __attribute__((aligned(16))) char k_lds1[HALF];
  __shared__ __attribute__((aligned(16))) char v_lds0[HALF];
  __shared__ __attribute__((aligned(16))) char v_lds1[HALF];
  __shared__ int list[MODE == kModeDense ? 1 : kMaxTiles];
  __shared__ int scan[kThreads];

  const int t = threadIdx.x, lane = t & 63, g = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  // Work items.  The long rows of every bank (query blocks ds .. tb-1: the text rows and a
  // ragged last video block, all dense) come first, dealt round-robin over the XCDs
  // (workgroup i runs on XCD i % 8): they start before the short ones and every XCD gets an
  // equal share.  The other rows follow in runs of 64 query blocks per XCD (about the
  // workgroups one XCD holds at once): the neighbouring Hilbert-ordered blocks in flight on
  // an XCD share many key tiles in its L2, and all XCDs together stay within ~512 blocks of
  // one bank, whose K/V images (58 MB at the HunyuanVideo shape) stay in the 256 MB
  // Infinity Cache.
  //
  // With a queue the workgroups are persistent (about two per CU) and claim their items:
  // XCD x holds the positions p = x, x + 8, x + 16, ... in that order, and a workgroup takes
  // the next one of its own XCD (one atomic increment) or, once those are all taken, of the
  // next XCD that still has one; it stops when every queue is empty.  XCDs that run faster
  // then process the slower ones' last items instead of idling.  Every increment below an
  // XCD's count claims a distinct position, so each item is processed exactly once.
  __shared__ int claimed;
  const int n_items = a.banks * a.tb;
  const bool persistent = a.queue != nullptr;
  for (int round = 0;; ++round) {
  int pos = blockIdx.x;
  if (persistent) {
    if (t == 0) {
      const int own = blockIdx.x & 7;
      int got = -1;
      for (int k = 0; k < 8 && got < 0; ++k) {
        const int x = (own + k) & 7;
        const int count = (n_items - x + 7) >> 3;  // positions on XCD x
        const int i = (int)atomicAdd(a.queue + kQueueStride * x, 1u);
        if (i < count) got = 8 * i + x;
      }
      claimed = got;  // -1: every queue is empty
    }
    __syncthreads();
    pos = __builtin_amdgcn_readfirstlane(claimed);
    if (pos < 0) break;
  } else if (round > 0) {
    break;
  }
  const int nlong = a.tb - a.ds, nshort = a.ds;
  const int n_long_items = a.banks * nlong;
  int bank, qt;
  if (pos < n_long_items) {
    bank = pos / nlong;
    qt = a.ds + pos % nlong;
  } else {
    const int lin = xcd_runs(pos - n_long_items, n_items - n_long_items, 64);
    bank = lin / nshort;
    qt = lin % nshort;
  }
  const int b = bank / a.heads, h = bank % a.heads;

  int nkeep = a.tb;
  if constexpr (MODE != kModeDense) {
    // Kept blocks in ascending order; in dense-head mode the other blocks follow them.
    const uint8_t* mrow = a.kmask + ((int64_t)bank * a.tb + qt) * a.tb;
    const int per = (a.tb + kThreads - 1) / kThreads;
    const int j0 = min(t * per, a.tb), j1 = min(j0 + per, a.tb);
    int cnt = 0;
    for (int j = j0; j < j1; ++j) cnt += mrow[j] != 0;
    scan[t] = cnt;
    __syncthreads();
    for (int off = 1; off < kThreads; off <<= 1) {
      const int v = t >= off ? scan[t - off] : 0;
      __syncthreads();
      scan[t] += v;
      __syncthreads();
    }
    int pos = scan[t] - cnt;
    nkeep = __builtin_amdgcn_readfirstlane(scan[kThreads - 1]);
    int npos = nkeep + (j0 - pos);  // blocks not kept before this thread's range
    // A kept ragged last block goes first, so its masked steps open the walk (in dense-head
    // mode the blocks that are not kept follow the kept ones, and the ragged block would
    // otherwise fall in the middle); every masked mode uses the same order.
    const bool lead = (a.n_tokens % kBlock) != 0 && mrow[a.tb - 1] != 0;
    for (int j = j0; j < j1; ++j) {
      if (mrow[j]) {
        list[lead ? (j == a.tb - 1 ? 0 : pos + 1) : pos] = j;
        ++pos;
      } else if (MODE == kModeDenseHead) {
        list[npos++] = j;
      }
    }
    __syncthreads();
  }
  const int nsub = MODE == kModeDenseHead ? 2 * a.tb : 2 * nkeep;  // 64-key sub-tiles

  // Sub-tile `it` = half (it & 1) of kept tile (it >> 1): its K rows and its V^T half are
  // each HALF contiguous bytes of the packed images, copied verbatim into LDS slot it & 1
  // by buffer loads into LDS (each lane moves 16 bytes; one wave instruction fills 1 KB in
  // lane order) over this bank's images, whose byte size bounds the buffer resource.
  const int bank_bytes = a.tb * G::kTileBytes;
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.kp + (int64_t)bank * a.tb * G::kTileElems), 0, bank_bytes, kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.vp + (int64_t)bank * a.tb * G::kTileElems), 0, bank_bytes, kBufferRsrcWord3);
  auto image = [&](int it) {  // byte offset of sub-tile `it` within the bank's images
    const int j = MODE == kModeDense ? (it >> 1) : list[it >> 1];
    return __builtin_amdgcn_readfirstlane(j * G::kTileBytes + (it & 1) * HALF);
  };
  auto copy = [&](__amdgpu_buffer_rsrc_t rs, int off, char* dst) {
#pragma unroll
    for (int i = 0; i < NDMA; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (lds_void*)(dst + 16 * kThreads * i + 1024 * wave), 16,
          16 * kThreads * i + 16 * t, off, 0, 0);
  };

  // Query group q of this wave: rows 32 q .. 32 q + 31 of the wave's kRowsPerWave.
  int row[kGroups], nat[kGroups];
  bool valid[kGroups];
#pragma unroll
  for (int q = 0; q < kGroups; ++q) {
    row[q] = qt * kBlock + wave * kRowsPerWave + 32 * q + l32;
    valid[q] = row[q] < a.n_tokens;
    nat[q] = valid[q] ? a.rowmap[row[q]] : 0;
  }
  if (nsub > 0) {
    copy(krs, image(0), k_lds0);
    copy(vrs, image(0), v_lds0);
  }
  if (nsub > 1) copy(krs, image(1), k_lds1);
  u32x4 qreg[kGroups][NS];
#pragma unroll
  for (int q = 0; q < kGroups; ++q) {
    const uint16_t* qrow = a.q + b * a.qsB + h * a.qsH + (int64_t)nat[q] * a.qsN;
#pragma unroll
    for (int s = 0; s < NS; ++s)
      qreg[q][s] = valid[q] ? *reinterpret_cast<const u32x4*>(qrow + 16 * s + 8 * g)
                            : u32x4{0u, 0u, 0u, 0u};
  }
  tile_barrier();

  float m[kGroups], mraw[kGroups], lsum[kGroups];
  const float inv_scale_log2 = 1.0f / a.scale_log2;
  f32x16 oacc[kGroups][NDT];
#pragma unroll
  for (int q = 0; q < kGroups; ++q) {
    m[q] = -INFINITY;
    mraw[q] = -INFINITY;
    lsum[q] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) oacc[q][dt] = f32x16{};
  }
  const bool ragged = (a.n_tokens % kBlock) != 0;

  // S^T (64 keys x 32 queries of each group) of the sub-tile whose K image is in `kl`.
  auto qk = [&](const char* kl, f32x16 (&s)[kGroups][2]) {
#pragma unroll
    for (int st = 0; st < NS; ++st)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const u32x4 ka = lds_load16(kl, G::k_off(32 * kt + l32, 2 * st + g));
#pragma unroll
        for (int q = 0; q < kGroups; ++q)
          s[q][kt] = T::mfma32(ka, qreg[q][st], st == 0 ? f32x16{} : s[q][kt]);
      }
  };
  // Keys past the sequence end in a sub-tile of the last (ragged) block.
  auto mask_tail = [&](f32x16 (&s)[kGroups][2], int it) {
    const int limit = a.n_tokens - ((a.tb - 1) * kBlock + 64 * (it & 1));
#pragma unroll
    for (int q = 0; q < kGroups; ++q)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int rr = 0; rr < 16; ++rr)
          if (32 * kt + mfma_row(rr, g) >= limit) s[q][kt][rr] = -INFINITY;
  };
  // Lazy running-max update of group q from a per-lane candidate raw score: moves only when
  // the row max grows by more than kRescaleSlack, rescaling O and l.  The test is on raw
  // scores against mraw = (m + slack) / (scale log2 e), kept with m (scale > 0).
  auto update_max = [&](int q, float mx) {
    const float pm = pair_max(mx);
    const bool grow = pm > mraw[q];
    if (__any(grow)) {
      const float mnew = grow ? pm * a.scale_log2 : m[q];
      const float alpha = __builtin_amdgcn_exp2f(m[q] - mnew);
      lsum[q] *= alpha;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) oacc[q][dt] *= alpha;
      m[q] = mnew;
      mraw[q] = (mnew + kRescaleSlack) * inv_scale_log2;
    }
  };
  auto row_max = [&](f32x16 (&s)[kGroups][2]) {
#pragma unroll
    for (int q = 0; q < kGroups; ++q) {
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) mx = __builtin_elementwise_maximum(mx, s[q][kt][rr]);
      update_max(q, mx);
    }
  };

  // Dense-head mode: the head branch of the kept blocks (the list's first 2 * nkeep
  // sub-tiles), stored from the running state once their last PV is done and before the
  // next sub-tile's scores may raise the running max -- the state head mode ends with.
  const int kept_end = 2 * nkeep;
  auto store_head = [&]() __attribute__((always_inline)) {
    if constexpr (MODE == kModeDenseHead) {
#pragma unroll
      for (int q = 0; q < kGroups; ++q) {
        const float lt = pair_sum(lsum[q]);
        if (valid[q])
          store_rows<T, D, kModeHead>(a, bank, b, h, row[q], nat[q], g, oacc[q], m[q], lt);
      }
    }
  };

  // One pipeline step, written as slices that the scheduler may not reorder: slice n reads
  // one LDS fragment (of slice n+2) and issues one MFMA per query group with the fragment
  // of slice n -- first the 2*NS of S_{it+1} (head-dimension chunk n/2, key tile n%2),
  // then the 4*NDT of PV_it (P chunk (kt, hh), O^T tile dt) -- plus a fixed share of VALU
  // work: while S_{it+1} runs, pairs of P_it = exp2(S_it scale log2e - m) values (two exp,
  // packed for the PV MFMAs); while PV_it runs, the row max over pairs of S_{it+1} scores.
  // The matrix core then works while the VALU does, instead of one after the other.
  // `it` is even at every call with parity tag 0 and odd with tag 1.
  auto step = [&](int it, f32x16 (&cur)[kGroups][2], f32x16 (&nxt)[kGroups][2], bool mask,
                  auto next_tag, auto parity_tag) __attribute__((always_inline)) {
    constexpr bool kNext = decltype(next_tag)::value;
    constexpr bool kOdd = decltype(parity_tag)::value;
    constexpr bool kSumCheck = D == 64;
    if (it + 1 < nsub) copy(vrs, image(it + 1), kOdd ? v_lds0 : v_lds1);
    if (it + 2 < nsub) copy(krs, image(it + 2), kOdd ? k_lds1 : k_lds0);
    const char* kl = kOdd ? k_lds0 : k_lds1;   // K_{it+1}
    const char* vl = kOdd ? v_lds1 : v_lds0;   // V_it
    constexpr int NQK = kNext ? 2 * NS : 0;  // S fragments of this step
    constexpr int NPV = 4 * NDT;             // PV fragments
    constexpr int NN = NQK + NPV;
    constexpr int NPAIR = 16 * kGroups;      // P pairs (16 per group)
    constexpr int PPS = kNext ? (NPAIR + NQK - 1) / (kNext ? NQK : 1) : NPAIR;  // P pairs per slice
    constexpr int MPS = 16 * kGroups / NPV;  // score pairs of the row max per PV slice
    auto frag = [&](int n) -> u32x4 {
      if (n < NQK) return lds_load16(kl, G::k_off(32 * (n & 1) + l32, 2 * (n >> 1) + g));
      const int i = n - NQK;
      return lds_load16(vl, G::vt_off(32 * (i % NDT) + l32, 2 * (i / NDT) + g));
    };
    unsigned w[kGroups][2][2][4];
    float part[kGroups][2];
    float mx[kGroups];
#pragma unroll
    for (int q = 0; q < kGroups; ++q) mx[q] = -INFINITY;
    u32x4 fr[3];
    fr[0] = frag(0);
    fr[1] = frag(1);
#pragma unroll
    for (int n = 0; n < NN; ++n) {
      if (n + 2 < NN) fr[(n + 2) % 3] = frag(n + 2);
      // P pairs first (the PV MFMAs need them); pair pr is pair pr / kGroups of group
      // pr % kGroups, so every group's chunk (kt, hh) is complete by the same slice.
      if (n * PPS < NPAIR) {
#pragma unroll
        for (int pr = n * PPS; pr < n * PPS + PPS && pr < NPAIR; ++pr) {
          const int q = pr % kGroups, pp = pr / kGroups;
          const int kt = pp >> 3, hh = (pp >> 2) & 1, e = 2 * (pp & 3);
          const float p0 = __builtin_amdgcn_exp2f(fmaf(cur[q][kt][8 * hh + e], a.scale_log2, -m[q]));
          const float p1 = __builtin_amdgcn_exp2f(fmaf(cur[q][kt][8 * hh + e + 1], a.scale_log2, -m[q]));
          part[q][kt] = (pp & 7) ? part[q][kt] + (p0 + p1) : p0 + p1;
          w[q][kt][hh][e >> 1] = pack2<T>(p0, p1);
        }
        if constexpr (kSumCheck) {
          // After the slice with the last pair, before any PV MFMA reads them: a lane whose
          // probabilities overflow the cap (or are not finite, as when m = -inf) redoes the
          // sub-tile against the raised running max, rescaling O and l first.
          if ((n + 1) * PPS >= NPAIR) {
            bool over = false;
#pragma unroll
            for (int q = 0; q < kGroups; ++q) over |= !(part[q][0] + part[q][1] <= kSumCap);
            if (__any(over)) {
              __builtin_amdgcn_sched_barrier(0);
#pragma unroll
              for (int q = 0; q < kGroups; ++q) {
                float mx = -INFINITY;
#pragma unroll
                for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                  for (int rr = 0; rr < 16; ++rr) mx = __builtin_elementwise_maximum(mx, cur[q][kt][rr]);
                const float mnew = pair_max(mx) * a.scale_log2;
                if (mnew > m[q]) {
                  const float alpha = __builtin_amdgcn_exp2f(m[q] - mnew);
                  lsum[q] *= alpha;
#pragma unroll
                  for (int dt = 0; dt < NDT; ++dt) oacc[q][dt] *= alpha;
                  m[q] = mnew;
                }
#pragma unroll
                for (int pp = 0; pp < 16; ++pp) {
                  const int kt = pp >> 3, hh = (pp >> 2) & 1, e = 2 * (pp & 3);
                  const float p0 = __builtin_amdgcn_exp2f(fmaf(cur[q][kt][8 * hh + e], a.scale_log2, -m[q]));
                  const float p1 = __builtin_amdgcn_exp2f(fmaf(cur[q][kt][8 * hh + e + 1], a.scale_log2, -m[q]));
                  part[q][kt] = (pp & 7) ? part[q][kt] + (p0 + p1) : p0 + p1;
                  w[q][kt][hh][e >> 1] = pack2<T>(p0, p1);
                }
              }
            }
          }
        }
      }
      if (n < NQK) {
        const int st = n >> 1, kt = n & 1;
#pragma unroll
        for (int q = 0; q < kGroups; ++q)
          nxt[q][kt] = T::mfma32(fr[n % 3], qreg[q][st], st == 0 ? f32x16{} : nxt[q][kt]);
        // S_{it+1} in the ragged last block: keys past the sequence end get -inf before the
        // row max reads them (a rare uniform branch, outside the scheduled slices).
        if (n == NQK - 1 && mask) {
          __builtin_amdgcn_sched_barrier(0);
          mask_tail(nxt, it + 1);
        }
      } else {
        const int i = n - NQK, kt = i / (2 * NDT), hh = (i / NDT) & 1, dt = i % NDT;
#pragma unroll
        for (int q = 0; q < kGroups; ++q) {
          const u32x4 pk = {w[q][kt][hh][0], w[q][kt][hh][1], w[q][kt][hh][2], w[q][kt][hh][3]};
          oacc[q][dt] = T::mfma32(fr[n % 3], pk, oacc[q][dt]);
        }
        if constexpr (kNext && !kSumCheck) {
          // Row max over MPS pairs of S_{it+1} scores (pair mp: group mp % kGroups).
#pragma unroll
          for (int mp = i * MPS; mp < (i + 1) * MPS; ++mp) {
            const int q = mp % kGroups, j = 2 * (mp / kGroups), kt2 = j >> 4, rr = j & 15;
            mx[q] = fmaxf(fmaxf(mx[q], nxt[q][kt2][rr]), nxt[q][kt2][rr + 1]);  // one v_max3_f32
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int q = 0; q < kGroups; ++q) lsum[q] += part[q][0] + part[q][1];
    if constexpr (MODE == kModeDenseHead) {
      if (it + 1 == kept_end) store_head();
    }
    if constexpr (kNext && !kSumCheck) {
#pragma unroll
      for (int q = 0; q < kGroups; ++q) update_max(q, mx[q]);
    }
    tile_barrier();
  };

  // True when sub-tile `it` of the list lies in the ragged last block.
  auto ragged_at = [&](int it) {
    const int j = MODE == kModeDense ? (it >> 1) : __builtin_amdgcn_readfirstlane(list[it >> 1]);
    return ragged && j == a.tb - 1;
  };
  f32x16 sa[kGroups][2], sb[kGroups][2];
  if (nsub > 0) {
    qk(k_lds0, sa);
    if (ragged_at(0)) mask_tail(sa, 0);
    row_max(sa);
    tile_barrier();  // step 0 overwrites K slot 0 (read just now)
  }
  using F = std::false_type;
  using Tr = std::true_type;
  // Steps go in pairs (even step: S in sa -> sb, odd step: sb -> sa) so each array keeps one
  // role.  Step it computes S of sub-tile it + 1, masked when that sub-tile lies in the ragged
  // last block: in the masked modes a kept ragged block goes first (sub-tiles 0 and 1), and in
  // dense mode, or in dense-head mode when the mask drops it, the ragged block goes last, so
  // only the first and the last two pairs are peeled and the main loop runs unmasked.  The
  // final step has no next sub-tile.
  if (MODE == kModeDenseHead && kept_end == 0) store_head();
  int it = 0;
  if constexpr (MODE != kModeDense) {
    if (nsub >= 4) {
      step(0, sa, sb, ragged_at(1), Tr{}, F{});
      step(1, sb, sa, ragged_at(2), Tr{}, Tr{});
      it = 2;
    }
  }
  for (; it + 4 < nsub; it += 2) {
    step(it, sa, sb, false, Tr{}, F{});
    step(it + 1, sb, sa, false, Tr{}, Tr{});
  }
  if (nsub - it >= 4) {
    step(it, sa, sb, false, Tr{}, F{});
    step(it + 1, sb, sa, ragged_at(it + 2), Tr{}, Tr{});
    it += 2;
  }
  if (nsub >= 2) {
    step(it, sa, sb, ragged_at(it + 1), Tr{}, F{});
    step(it + 1, sb, sa, false, F{}, Tr{});
  }

  constexpr int kStore = MODE == kModeDenseHead ? kModeDense : MODE;
#pragma unroll
  for (int q = 0; q < kGroups; ++q) {
    const float lt = pair_sum(lsum[q]);  // lanes l and l ^ 32 share one row: both valid or not
    if (valid[q]) store_rows<T, D, kStore>(a, bank, b, h, row[q], nat[q], g, oacc[q], m[q], lt);
  }
  __syncthreads();  // every wave is done with the LDS slots, the list and `claimed`
  }  // items
}

// Workgroups of a persistent launch: two per CU (the attention kernel's occupancy), no
// more than there are items.
static int persistent_grid(int items) {
  int device = 0, cus = 0;
  if (hipGetDevice(&device) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
      cus < 1)
    cus = 256;
  return items < 2 * cus ? items : 2 * cus;
}

template <class T, int D>
static hipError_t launch_attention(const AttnArgs& a, int mode, hipStream_t s) {
  const int items = a.banks * a.tb;
  const dim3 grid((unsigned)(a.queue != nullptr ? persistent_grid(items) : items)), block(kThreads);
  switch (mode) {
    case kModeHead: hipLaunchKernelGGL((attention_kernel<T, D, kModeHead>), grid, block, 0, s, a); break;
    case kModeDense: hipLaunchKernelGGL((attention_kernel<T, D, kModeDense>), grid, block, 0, s, a); break;
    case kModeDenseHead: hipLaunchKernelGGL((attention_kernel<T, D, kModeDenseHead>), grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL((attention_kernel<T, D, kModeMerge>), grid, block, 0, s, a); break;
  }
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void zero_words_kernel(unsigned* p, int n) {
  for (int i = threadIdx.x; i < n; i += 256) p[i] = 0u;
}

hipError_t run_zero_words(unsigned* p, int n, hipStream_t s) {
  hipLaunchKernelGGL(zero_words_kernel, dim3(1), dim3(256), 0, s, p, n);
  return hipGetLastError();
}

hipError_t run_attention(const AttnArgs& a, int dtype, int dim, int mode, hipStream_t s) {
  if (dtype == BF16::code)
    return dim == 128 ? launch_attention<BF16, 128>(a, mode, s) : launch_attention<BF16, 64>(a, mode, s);
  return dim == 128 ? launch_attention<F16, 128>(a, mode, s) : launch_attention<F16, 64>(a, mode, s);
}

}  // namespace recap
