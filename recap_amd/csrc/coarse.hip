// Stage 3: the corrected coarse tail over each query block's omitted key blocks.
//
// Math of recap/kernels/coarse_tail.py:79-186 with the wrapper steps of :224-312 and
// recap/sparse/attention.py:187-195, 224-230 fused in:
//   qsq   = (U^T q)^2      in the query type  (recap/sparse/closure.py:84-86)
//   drift = s C_vk q       in the query type  (recap/sparse/closure.py:89-93)
//   l_j   = s q.kbar_j + ln n_j + [s^2 qsq.w_j <= theta^2] (s^2/2) qsq.w_j
//   out   = softmax(l) . vbar  (+ g * drift, g = gated share of the mass), lse = m + ln l
// over the omitted blocks j (~partition[i, j]); the omitted list is compacted in LDS
// from the partition row, so no host-side planning or synchronisation is needed
// (recap/sparse/planner.py:24-27 is the host sync this removes).
//
// One workgroup = one (bank, 128-row query block), 4 waves x 32 rows.  The three
// contractions per 32-block tile (q.kbar, qsq.w, p.vbar) run on 32x32x16 MFMA with the
// same register-resident layout trick as the attention kernel: the fp32 result of one
// MFMA is the B operand of the next, and the tables' columns (w) or rows (vbar^T in LDS)
// are stored in the matching swap23 order.  Also writes per-block partial sums of
// (gl - gl_ref) for the per-bank drift centre (recap/operator.py:148-150).
#include "kernels.hpp"

namespace recap {

constexpr int kMaxVideoBlocks = 4096;

template <class T, int D>
__global__ __launch_bounds__(256, 2) void coarse_kernel(CoarseArgs a) {
#pragma clang fp contract(off)
  using G = TileGeom<D>;
  constexpr int NS = D / 16, NDT = D / 32, NCH = D / 8;
  constexpr int kMatBytes = D * D * 2;
  constexpr int kTabBytes = 32 * D * 2;
  constexpr int kBuf = kMatBytes > 3 * kTabBytes ? kMatBytes : 3 * kTabBytes;
  __shared__ __attribute__((aligned(16))) char buf[kBuf];
  __shared__ uint16_t list[kMaxVideoBlocks];
  __shared__ int scan[256];
  __shared__ float wsum[4];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, g = lane >> 5, l32 = lane & 31;
  const int lin = xcd_linear(blockIdx.x, a.banks * a.qtiles);
  const int bank = lin / a.qtiles, qt = lin % a.qtiles;
  const int b = bank / a.heads, h = bank % a.heads;

  // Omitted blocks of this query block, in increasing order.
  int n_omit;
  {
    const uint8_t* prow = a.partition + ((int64_t)bank * a.nb + qt) * a.nb;
    const int per = (a.nb + 255) / 256;
    const int j0 = min(t * per, a.nb), j1 = min(j0 + per, a.nb);
    int cnt = 0;
    for (int j = j0; j < j1; ++j) cnt += prow[j] == 0;
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
      if (prow[j] == 0) list[pos++] = (uint16_t)j;
    n_omit = scan[255];
  }

  // Stage U^T (query type, [D][D]) into LDS.
  {
    const uint16_t* us = a.u_t + (int64_t)bank * D * D;
    for (int cc = t; cc < D * NCH; cc += 256) {
      const int row = cc / NCH, c = cc % NCH;
      *reinterpret_cast<u32x4*>(buf + G::k_off(row, c)) =
          *reinterpret_cast<const u32x4*>(us + row * D + c * 8);
    }
  }

  const int r = qt * kBlock + wave * 32 + l32;  // always < rows
  const int nat = a.rowmap[r];
  u32x4 qreg[NS];
  {
    const uint16_t* qrow = a.q + b * a.sB + h * a.sH + (int64_t)nat * a.sN;
#pragma unroll
    for (int s = 0; s < NS; ++s) qreg[s] = *reinterpret_cast<const u32x4*>(qrow + 16 * s + 8 * g);
  }
  __syncthreads();

  // qsq in the B-operand layout of the quadratic form.
  u32x4 qsq_pk[NDT][2];
#pragma unroll
  for (int ot = 0; ot < NDT; ++ot) {
    f32x16 acc = f32x16{};
#pragma unroll
    for (int s = 0; s < NS; ++s)
      acc = T::mfma32(lds_load16(buf, G::k_off(32 * ot + l32, 2 * s + g)), qreg[s], acc);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      unsigned w[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float x0 = T::to_f(T::from_f(acc[8 * hh + e]));
        const float x1 = T::to_f(T::from_f(acc[8 * hh + e + 1]));
        w[e >> 1] = pack2<T>(x0 * x0, x1 * x1);
      }
      qsq_pk[ot][hh] = u32x4{w[0], w[1], w[2], w[3]};
    }
  }

  const float s32 = a.scale;
  const float ssq = (float)((double)a.scale * (double)a.scale);
  const float half = (float)(0.5 * (double)a.scale * (double)a.scale);
  const float thsq = (float)((double)a.theta * (double)a.theta);
  const float ln_full = logf((float)kBlock);
  const float ln_last = logf((float)(a.n_video - kBlock * (a.nb - 1)));

  char* kb_lds = buf;
  char* w_lds = buf + kTabBytes;
  char* vt_lds = buf + 2 * kTabBytes;
  float m = -INFINITY, lsum = 0.0f, gsum = 0.0f;
  f32x16 oacc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) oacc[dt] = f32x16{};

  for (int base = 0; base < n_omit; base += 32) {
    __syncthreads();
    for (int cc = t; cc < 32 * NCH; cc += 256) {
      const int slot = cc / NCH, c = cc % NCH;
      const bool valid = base + slot < n_omit;
      const int64_t row = (int64_t)bank * a.nb + (valid ? list[base + slot] : 0);
      const u32x4 zero = {0u, 0u, 0u, 0u};
      const u32x4 kv = valid ? *reinterpret_cast<const u32x4*>(a.kbar + row * D + 8 * c) : zero;
      const u32x4 wv = valid ? *reinterpret_cast<const u32x4*>(a.w + row * D + 8 * c) : zero;
      const u32x4 vv = valid ? *reinterpret_cast<const u32x4*>(a.vbar + row * D + 8 * c) : zero;
      *reinterpret_cast<u32x4*>(kb_lds + G::k_off(slot, c)) = kv;
      *reinterpret_cast<u32x4*>(w_lds + G::k_off(slot, c)) = wv;
      const int pos = swap23(slot);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = 8 * c + e;
        const uint16_t hv = (uint16_t)((e & 1) ? vv[e >> 1] >> 16 : vv[e >> 1] & 0xffff);
        const int off = d * 64 + ((((pos >> 3) ^ ((d >> 2) & 3))) << 4) + ((pos & 7) << 1);
        *reinterpret_cast<uint16_t*>(vt_lds + off) = hv;
      }
    }
    __syncthreads();

    f32x16 sacc = f32x16{}, wacc = f32x16{};
#pragma unroll
    for (int s = 0; s < NS; ++s) sacc = T::mfma32(lds_load16(kb_lds, G::k_off(l32, 2 * s + g)), qreg[s], sacc);
#pragma unroll
    for (int ot = 0; ot < NDT; ++ot)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
        wacc = T::mfma32(lds_load16(w_lds, G::k_off(l32, 4 * ot + 2 * hh + g)), qsq_pk[ot][hh], wacc);

    float sc[16];
    bool gate[16];
    float mx = -INFINITY;
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      const int idx = base + mfma_row(rr, g);
      if (idx < n_omit) {
        const int j = list[idx];
        float v = sacc[rr] * s32;
        v = v + (j == a.nb - 1 ? ln_last : ln_full);
        const float quad = wacc[rr];
        gate[rr] = quad * ssq <= thsq;
        v = v + (gate[rr] ? quad * half : 0.0f);
        sc[rr] = v;
      } else {
        sc[rr] = -INFINITY;
        gate[rr] = false;
      }
      mx = fmaxf(mx, sc[rr]);
    }
    mx = pair_max(mx);
    const float mnew = fmaxf(m, mx);
    const float alpha = expf(m - mnew);
    lsum *= alpha;
    gsum *= alpha;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) oacc[dt] *= alpha;
    m = mnew;
    u32x4 pk[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      unsigned w[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float p0 = expf(sc[8 * hh + e] - mnew);
        const float p1 = expf(sc[8 * hh + e + 1] - mnew);
        lsum += p0;
        lsum += p1;
        gsum += gate[8 * hh + e] ? p0 : 0.0f;
        gsum += gate[8 * hh + e + 1] ? p1 : 0.0f;
        w[e >> 1] = pack2<T>(p0, p1);
      }
      pk[hh] = u32x4{w[0], w[1], w[2], w[3]};
    }
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const int d = 32 * dt + l32;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int off = d * 64 + ((((2 * hh + g) ^ ((d >> 2) & 3))) << 4);
        oacc[dt] = T::mfma32(lds_load16(vt_lds, off), pk[hh], oacc[dt]);
      }
    }
  }

  // Value drift s C_vk q in the output layout: stage C_vk over the tables' LDS.
  __syncthreads();
  {
    const uint16_t* cs = a.cvk + (int64_t)bank * D * D;
    for (int cc = t; cc < D * NCH; cc += 256) {
      const int row = cc / NCH, c = cc % NCH;
      *reinterpret_cast<u32x4*>(buf + G::k_off(row, c)) =
          *reinterpret_cast<const u32x4*>(cs + row * D + c * 8);
    }
  }
  __syncthreads();

  const float l = pair_sum(lsum);
  const float gs = pair_sum(gsum);
  const bool has_tail = l > 0.0f;
  const float safe_l = fmaxf(l, 1.0e-30f);
  const float gfrac = T::to_f(T::from_f(has_tail ? gs / safe_l : 0.0f));
  const int64_t ri = (int64_t)bank * a.rows + r;
  uint16_t* gorow = a.go + ri * D;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    f32x16 dacc = f32x16{};
#pragma unroll
    for (int s = 0; s < NS; ++s)
      dacc = T::mfma32(lds_load16(buf, G::k_off(32 * dt + l32, 2 * s + g)), qreg[s], dacc);
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float o = has_tail ? T::to_f(T::from_f(oacc[dt][4 * q4 + e] / safe_l)) : 0.0f;
        const float dv = T::to_f(T::from_f(T::to_f(T::from_f(dacc[4 * q4 + e])) * a.scale));
        const float gd = T::to_f(T::from_f(gfrac * dv));
        v[e] = o + gd;
      }
      *reinterpret_cast<u32x2*>(gorow + 32 * dt + 8 * q4 + 4 * g) =
          u32x2{pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3])};
    }
  }
  const float lse = has_tail ? m + logf(l) : -INFINITY;
  if (g == 0) a.gl[ri] = lse;
  if (a.glref != nullptr) {
    const float diff = half_wave_sum(lse - a.glref[ri]);
    if (lane == 0) wsum[wave] = diff;
    __syncthreads();
    if (t == 0) a.drift_part[(int64_t)bank * a.qtiles + qt] = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
  }
}

template <class T, int D>
static hipError_t launch_coarse(const CoarseArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((coarse_kernel<T, D>), dim3((unsigned)(a.banks * a.qtiles)), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t run_coarse(const CoarseArgs& a, int dtype, int dim, hipStream_t s) {
  if (dtype == BF16::code) return dim == 128 ? launch_coarse<BF16, 128>(a, s) : launch_coarse<BF16, 64>(a, s);
  return dim == 128 ? launch_coarse<F16, 128>(a, s) : launch_coarse<F16, 64>(a, s);
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
