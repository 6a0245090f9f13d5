// Stage 4 at a refresh: capture the refinement of the tail (recap/kernels/detail_cache.py:
// 64-186, 304-379).  For video rows r < R, with the dense output / LSE read at the native
// row rowmap[r] (= video_offset + permutation[r]):
//   ratio = min(exp(min(lh - lf, 0)), 1 - 1e-6)
//   D     = clamp((of - ratio oh) / (1 - ratio) - go, +-6e4), 0 where ratio > 1 - 1e-3
//   DL    = clamp(lf + ln(1 - ratio) - gl, +-30)
// With a previous refinement it first rebuilds the sparse output that refinement gives
// (drift weight included) and accumulates sum (old - of)^2 and sum of^2.  The reference
// adds them with float atomics; here each workgroup writes a partial pair and sum_pairs
// adds them in a fixed order.  Elementwise, HBM-bound, 16-byte accesses.
#include <mutex>

#include "kernels.hpp"

namespace recap {

template <class T, int D>
__global__ __launch_bounds__(256) void capture_kernel(CaptureArgs a) {
  constexpr int TPR = D / 8, RPB = 256 / TPR;
  __shared__ float red[2][4];
  const int blocks = a.rows / RPB;
  const int bank = blockIdx.x / blocks, blk = blockIdx.x % blocks;
  const int b = bank / a.heads, h = bank % a.heads;
  const int t = threadIdx.x, c = t % TPR;
  const int r = blk * RPB + t / TPR;
  const int nat = a.rowmap[r];
  const int64_t ri = (int64_t)bank * a.rows + r;
  const float lf = a.lf[(int64_t)bank * a.n_tokens + nat];
  const float lh = a.lh[(int64_t)bank * a.n_tokens + r];
  const float glv = a.gl[ri];
  float ratio = expf(fminf(lh - lf, 0.0f));
  ratio = fminf(ratio, 1.0f - 1.0e-6f);
  const float den = 1.0f - ratio;

  const u32x4 ofw = *reinterpret_cast<const u32x4*>(a.of + b * a.osB + h * a.osH + (int64_t)nat * a.osN + 8 * c);
  const u32x4 ohw = *reinterpret_cast<const u32x4*>(a.oh + ((int64_t)bank * a.n_tokens + r) * D + 8 * c);
  const u32x4 gow = *reinterpret_cast<const u32x4*>(a.go + ri * D + 8 * c);
  float of[8], oh[8], go[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int sh = (e & 1) * 16;
    of[e] = T::to_f((uint16_t)(ofw[e >> 1] >> sh));
    oh[e] = T::to_f((uint16_t)(ohw[e >> 1] >> sh));
    go[e] = T::to_f((uint16_t)(gow[e >> 1] >> sh));
  }

  const bool validate = a.glref != nullptr;
  float err2 = 0.0f, ref2 = 0.0f;
  if (validate) {
    const u32x4 dw = *reinterpret_cast<const u32x4*>(a.det + ri * D + 8 * c);
    const float old_dl = a.dl[ri];
    const float admit = expf(-fabsf(glv - a.glref[ri] - a.center[bank]));
    const float cl = glv + old_dl;
    const float tc = fmaxf(glv, cl);
    const float sm = (1.0f - admit) * expf(glv - tc);
    const float cm = admit * expf(cl - tc);
    const float tden = fmaxf(sm + cm, 1.0e-30f);
    const float tl = tc + logf(tden);
    const float common = fmaxf(lh, tl);
    const float wh = expf(lh - common), wt = expf(tl - common);
    const float mden = fmaxf(wh + wt, 1.0e-30f);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float det = f16_to_f((uint16_t)(dw[e >> 1] >> ((e & 1) * 16)));
      const float to = (go[e] * sm + (go[e] + det) * cm) / tden;
      const float old = (oh[e] * wh + to * wt) / mden;
      err2 += (old - of[e]) * (old - of[e]);
      ref2 += of[e] * of[e];
    }
    __syncthreads();  // every old value of this block's rows is read before any write
  }

  unsigned w[4];
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    float v[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const float tail = (of[e + u] - ratio * oh[e + u]) / den;
      float cached = fmaxf(fminf(tail - go[e + u], 6.0e4f), -6.0e4f);
      v[u] = ratio > 1.0f - 1.0e-3f ? 0.0f : cached;
    }
    w[e >> 1] = (unsigned)f_to_f16(v[0]) | ((unsigned)f_to_f16(v[1]) << 16);
  }
  *reinterpret_cast<u32x4*>(a.det + ri * D + 8 * c) = u32x4{w[0], w[1], w[2], w[3]};
  if (c == 0) a.dl[ri] = fmaxf(fminf(lf + logf(den) - glv, 30.0f), -30.0f);

  if (validate) {
    err2 = wave_sum(err2);
    ref2 = wave_sum(ref2);
    const int wave = t >> 6;
    if ((t & 63) == 0) { red[0][wave] = err2; red[1][wave] = ref2; }
    __syncthreads();
    if (t == 0) {
      float* out = a.stat_part + 2 * (int64_t)blockIdx.x;
      out[0] = ((red[0][0] + red[0][1]) + red[0][2]) + red[0][3];
      out[1] = ((red[1][0] + red[1][1]) + red[1][2]) + red[1][3];
    }
  }
}

template <class T, int D>
static hipError_t launch_capture(const CaptureArgs& a, int* blocks_per_bank, hipStream_t s) {
  constexpr int RPB = 256 / (D / 8);
  *blocks_per_bank = a.rows / RPB;
  hipLaunchKernelGGL((capture_kernel<T, D>), dim3((unsigned)(a.banks * (a.rows / RPB))), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t run_capture(const CaptureArgs& a, int dtype, int dim, int* blocks_per_bank, hipStream_t s) {
  if (dtype == BF16::code)
    return dim == 128 ? launch_capture<BF16, 128>(a, blocks_per_bank, s) : launch_capture<BF16, 64>(a, blocks_per_bank, s);
  return dim == 128 ? launch_capture<F16, 128>(a, blocks_per_bank, s) : launch_capture<F16, 64>(a, blocks_per_bank, s);
}

// ---------------------------------------------------------------------------------------
// Static scratch of the allocation-free capture (recap_refresh_capture_noalloc): the
// per-workgroup validation pairs live in this file-scope device array instead of a caller
// workspace.  Each GPU holds its own copy until the process ends; its address on a device
// is looked up once, with that device current, and kept per device.  In host code the
// array's name is only a host-side stand-in, so kernels and copies get the looked-up
// address, never the name.
__device__ __align__(256) float capture_scratch[2 * kCaptureScratchPairs];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
float* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

hipError_t capture_scratch_pointer(float** out) {
  int device = -1;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return e;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (g_scratch_ptr[device] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(capture_scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[device] = static_cast<float*>(ptr);
  }
  *out = g_scratch_ptr[device];
  return hipSuccess;
}

// out2 = fixed-order sums of n (a, b) pairs: thread t adds pairs t, t + 1024, t + 2048, ...
// in turn (coalesced loads), then a fixed tree over the threads.
constexpr int kSumThreads = 1024;

__global__ __launch_bounds__(kSumThreads) void sum_pairs_kernel(const float* part, int n, float* out2) {
  __shared__ float ra[kSumThreads], rb[kSumThreads];
  const int t = threadIdx.x;
  const f32x2* pairs = reinterpret_cast<const f32x2*>(part);
  float sa = 0.0f, sb = 0.0f;
#pragma unroll 8
  for (int i = t; i < n; i += kSumThreads) {
    const f32x2 v = pairs[i];
    sa += v[0];
    sb += v[1];
  }
  ra[t] = sa;
  rb[t] = sb;
  __syncthreads();
  for (int h = kSumThreads / 2; h >= 1; h >>= 1) {
    if (t < h) { ra[t] += ra[t + h]; rb[t] += rb[t + h]; }
    __syncthreads();
  }
  if (t == 0) { out2[0] = ra[0]; out2[1] = rb[0]; }
}

hipError_t run_sum_pairs(const float* part, int n, float* out2, hipStream_t s) {
  hipLaunchKernelGGL(sum_pairs_kernel, dim3(1), dim3(kSumThreads), 0, s, part, n, out2);
  return hipGetLastError();
}

}  // namespace recap
