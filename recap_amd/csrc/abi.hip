// extern "C" entry points of librecap_hip.so (declared in include/recap_hip.h): host-side
// argument validation, derived geometry, and dispatch to the kernel launchers.
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <string>
#include <utility>
#include <vector>

#include "../../include/recap_hip.h"

#include <cmath>
#include "kernels.hpp"

using namespace recap;

namespace {

thread_local std::string g_error = "no error";

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(RECAP_EHIP, "%s: %s", what, hipGetErrorString(e));
  return RECAP_OK;
}

#define REQUIRE(cond, ...)                               \
  do {                                                   \
    if (!(cond)) return fail(RECAP_EINVAL, __VA_ARGS__); \
  } while (0)

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

struct Geom {
  int64_t nb, tb, ds, rows;
};

Geom geometry(int64_t n_tokens, int64_t n_video) {
  Geom g;
  g.nb = (n_video + kBlock - 1) / kBlock;
  g.tb = (n_tokens + kBlock - 1) / kBlock;
  const bool shared = (n_video % kBlock) != 0 && n_tokens > n_video;
  g.ds = shared ? g.nb - 1 : g.nb;
  g.rows = (n_video / kBlock) * kBlock;
  return g;
}

int check_common(int dtype, int64_t dim) {
  REQUIRE(dtype == RECAP_BF16 || dtype == RECAP_F16, "dtype %d is not RECAP_BF16 or RECAP_F16", dtype);
  REQUIRE(dim == 64 || dim == 128, "head dim %lld unsupported (64 or 128)", (long long)dim);
  return RECAP_OK;
}

int check_tokens(int64_t n_tokens, int64_t n_video) {
  REQUIRE(n_video >= 1, "n_video must be positive");
  REQUIRE(n_tokens >= n_video, "n_tokens %lld < n_video %lld", (long long)n_tokens, (long long)n_video);
  REQUIRE(n_tokens < (1ll << 31) / kBlock, "n_tokens too large");
  return RECAP_OK;
}

int check_qkv(const char* name, const void* p, int64_t batch, int64_t heads, int64_t sb,
              int64_t sh, int64_t sn) {
  REQUIRE(p != nullptr, "%s is NULL", name);
  REQUIRE(batch >= 1 && heads >= 1, "%s: batch and heads must be positive", name);
  REQUIRE(aligned16(p), "%s is not 16-byte aligned", name);
  REQUIRE(sb % 8 == 0 && sh % 8 == 0 && sn % 8 == 0 && sb >= 0 && sh >= 0 && sn > 0,
          "%s strides (%lld, %lld, %lld) must be non-negative multiples of 8 elements", name,
          (long long)sb, (long long)sh, (long long)sn);
  return RECAP_OK;
}

// Softmax scale of an attention launch: positive and finite (the kernels' running max is
// taken over raw scores and scaled afterwards, which needs scale > 0).
int set_scale(AttnArgs& a, float scale) {
  REQUIRE(std::isfinite(scale) && scale > 0.0f, "scale must be positive and finite, got %g",
          (double)scale);
  a.scale_log2 = scale * kLog2e;
  return RECAP_OK;
}

#define CHECK(expr)                 \
  do {                              \
    const int _rc = (expr);         \
    if (_rc != RECAP_OK) return _rc; \
  } while (0)

// Optional claim queues of an attention launch: zeroed on the stream (a fill kernel, so a
// captured graph records no memset) right before the launch that uses them.
int set_queue(AttnArgs& a, uint32_t* queue, hipStream_t s) {
  a.queue = nullptr;
  if (queue == nullptr) return RECAP_OK;
  REQUIRE(aligned16(queue), "work_queue must be 16-byte aligned");
  CHECK(hip_status(run_zero_words(queue, kQueueWords, s), "work_queue reset"));
  a.queue = queue;
  return RECAP_OK;
}

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace

extern "C" {

int recap_abi_version(void) { return RECAP_ABI_VERSION; }

const char* recap_last_error(void) { return g_error.c_str(); }

// J. Skilling, "Programming the Hilbert curve" (AIP Conf. Proc. 707, 2004): axes to
// transposed Hilbert index, x as the leading axis; the transposed bits are interleaved
// most significant first into one key, and native indices are ordered by key.
int recap_hilbert_permutation(int64_t frames, int64_t height, int64_t width, int64_t* out) {
  REQUIRE(out != nullptr, "out is NULL");
  REQUIRE(frames >= 1 && height >= 1 && width >= 1, "grid must be positive");
  const int64_t largest = std::max(frames, std::max(height, width));
  int bits = 0;
  while ((int64_t(1) << bits) < largest) ++bits;
  bits = std::max(bits, 1);
  REQUIRE(bits <= 21, "grid too large for a 63-bit Hilbert key");
  const int64_t n = frames * height * width;
  std::vector<std::pair<uint64_t, int64_t>> keyed((size_t)n);
  const uint64_t top = uint64_t(1) << (bits - 1);
  int64_t idx = 0;
  for (int64_t t = 0; t < frames; ++t)
    for (int64_t y = 0; y < height; ++y)
      for (int64_t x = 0; x < width; ++x, ++idx) {
        uint64_t X[3] = {(uint64_t)x, (uint64_t)y, (uint64_t)t};
        for (uint64_t q = top; q > 1; q >>= 1) {
          const uint64_t low = q - 1;
          for (int i = 0; i < 3; ++i) {
            if (X[i] & q) {
              X[0] ^= low;
            } else {
              const uint64_t swap = (X[0] ^ X[i]) & low;
              X[0] ^= swap;
              X[i] ^= swap;
            }
          }
        }
        X[1] ^= X[0];
        X[2] ^= X[1];
        uint64_t flip = 0;
        for (uint64_t q = top; q > 1; q >>= 1)
          if (X[2] & q) flip ^= q - 1;
        for (int i = 0; i < 3; ++i) X[i] ^= flip;
        uint64_t key = 0;
        for (int b = bits - 1; b >= 0; --b)
          for (int i = 0; i < 3; ++i) key = (key << 1) | ((X[i] >> b) & 1);
        keyed[(size_t)idx] = {key, t * height * width + y * width + x};
      }
  std::stable_sort(keyed.begin(), keyed.end(),
                   [](const auto& a, const auto& b) { return a.first < b.first; });
  for (int64_t i = 0; i < n; ++i) out[i] = keyed[(size_t)i].second;
  return RECAP_OK;
}

int recap_pool_blocks(const void* x, int dtype, int64_t batch, int64_t heads, int64_t dim,
                      int64_t stride_b, int64_t stride_h, int64_t stride_n,
                      const int32_t* rowmap, int64_t n_tokens, int64_t n_video,
                      float* means, void* stream) {
  CHECK(check_common(dtype, dim));
  CHECK(check_tokens(n_tokens, n_video));
  CHECK(check_qkv("x", x, batch, heads, stride_b, stride_h, stride_n));
  REQUIRE(rowmap && means, "rowmap and means must be non-NULL");
  const Geom g = geometry(n_tokens, n_video);
  PackPoolArgs a{};
  a.x0 = static_cast<const uint16_t*>(x);
  a.sB0 = stride_b; a.sH0 = stride_h; a.sN0 = stride_n;
  a.rowmap = rowmap;
  a.heads = (int)heads; a.banks = (int)(batch * heads);
  a.n_tokens = (int)n_tokens; a.n_video = (int)n_video;
  a.nb = (int)g.nb; a.tb = (int)g.nb;  // video blocks only
  a.mean0 = means;
  return hip_status(run_pack_pool(a, dtype, (int)dim, false, as_stream(stream)), "pool_blocks launch");
}

int recap_kv_pack(const void* k, const void* v, int dtype, int64_t batch, int64_t heads,
                  int64_t dim, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_n,
                  int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_n,
                  const int32_t* rowmap, int64_t n_tokens, int64_t n_video, void* k_tiles,
                  void* vt_tiles, float* k_means, float* v_means, void* stream) {
  CHECK(check_common(dtype, dim));
  CHECK(check_tokens(n_tokens, n_video));
  CHECK(check_qkv("k", k, batch, heads, k_stride_b, k_stride_h, k_stride_n));
  CHECK(check_qkv("v", v, batch, heads, v_stride_b, v_stride_h, v_stride_n));
  REQUIRE(rowmap && k_tiles && vt_tiles && k_means && v_means, "NULL output or rowmap");
  REQUIRE(aligned16(k_tiles) && aligned16(vt_tiles), "tile buffers must be 16-byte aligned");
  const Geom g = geometry(n_tokens, n_video);
  PackPoolArgs a{};
  a.x0 = static_cast<const uint16_t*>(k);
  a.sB0 = k_stride_b; a.sH0 = k_stride_h; a.sN0 = k_stride_n;
  a.x1 = static_cast<const uint16_t*>(v);
  a.sB1 = v_stride_b; a.sH1 = v_stride_h; a.sN1 = v_stride_n;
  a.rowmap = rowmap;
  a.heads = (int)heads; a.banks = (int)(batch * heads);
  a.n_tokens = (int)n_tokens; a.n_video = (int)n_video;
  a.nb = (int)g.nb; a.tb = (int)g.tb;
  a.kp = static_cast<uint16_t*>(k_tiles); a.vp = static_cast<uint16_t*>(vt_tiles);
  a.mean0 = k_means; a.mean1 = v_means;
  return hip_status(run_pack_pool(a, dtype, (int)dim, true, as_stream(stream)), "kv_pack launch");
}

int recap_block_scores(const float* q_means, const float* k_means, int64_t banks,
                       int64_t n_blocks, int64_t dim, float scale, float* scores, void* stream) {
  REQUIRE(q_means && k_means && scores, "NULL pointer");
  REQUIRE(dim == 64 || dim == 128, "head dim %lld unsupported", (long long)dim);
  REQUIRE(std::isfinite(scale) && scale > 0.0f, "scale must be positive and finite, got %g",
          (double)scale);
  REQUIRE(banks >= 1 && n_blocks >= 1 && n_blocks <= 65535, "bad banks/n_blocks");
  ScoreArgs a{q_means, k_means, (int)banks, (int)n_blocks, (int)dim, scale, scores};
  return hip_status(run_block_scores(a, as_stream(stream)), "block_scores launch");
}

int recap_topk_blocks(const float* scores, int64_t banks, int64_t n_blocks, int64_t keep,
                      int force_last, uint8_t* partition, void* stream) {
  REQUIRE(scores && partition, "NULL pointer");
  REQUIRE(banks >= 1 && n_blocks >= 1, "bad banks/n_blocks");
  REQUIRE(n_blocks <= 4096, "n_blocks %lld exceeds 4096", (long long)n_blocks);
  REQUIRE(keep >= 1 && keep <= n_blocks, "keep %lld outside 1..%lld", (long long)keep, (long long)n_blocks);
  TopkArgs a{scores, (int)banks, (int)n_blocks, (int)keep, force_last ? 1 : 0, partition};
  return hip_status(run_topk(a, as_stream(stream)), "topk launch");
}

int recap_kernel_block_mask(const uint8_t* partition, int64_t banks, int64_t n_tokens,
                            int64_t n_video, uint8_t* kernel_mask, void* stream) {
  REQUIRE(partition && kernel_mask, "NULL pointer");
  CHECK(check_tokens(n_tokens, n_video));
  REQUIRE(banks >= 1, "bad banks");
  const Geom g = geometry(n_tokens, n_video);
  KmaskArgs a{partition, (int)banks, (int)g.nb, (int)g.tb, (int)g.ds, kernel_mask};
  return hip_status(run_kernel_mask(a, as_stream(stream)), "kernel_mask launch");
}

static int64_t align256(int64_t bytes) { return (bytes + 255) / 256 * 256; }

int64_t recap_pool_select_workspace_size(int64_t banks, int64_t n_blocks, int64_t dim) {
  if (banks < 1 || n_blocks < 1 || dim < 1) return -1;
  return align256(banks * n_blocks * dim * 4) + align256(banks * n_blocks * n_blocks * 4);
}

int recap_pool_select(const void* q, int dtype, int64_t batch, int64_t heads, int64_t dim,
                      int64_t stride_b, int64_t stride_h, int64_t stride_n,
                      const int32_t* rowmap, int64_t n_tokens, int64_t n_video,
                      const float* k_means, float scale, double density, void* workspace,
                      int64_t workspace_bytes, uint8_t* partition, uint8_t* kernel_mask,
                      void* stream) {
  CHECK(check_tokens(n_tokens, n_video));
  REQUIRE(k_means && workspace && partition && kernel_mask, "NULL pointer");
  REQUIRE(density > 0.0 && density < 1.0, "density %g outside (0, 1)", density);
  REQUIRE(std::isfinite(scale) && scale > 0.0f, "scale must be positive and finite, got %g",
          (double)scale);
  REQUIRE(batch >= 1 && heads >= 1, "bad batch/heads");
  const Geom g = geometry(n_tokens, n_video);
  // every check of the four stages is made here, before the first of them launches
  CHECK(check_common(dtype, dim));
  REQUIRE(g.nb <= 4096, "too many video blocks (%lld > 4096)", (long long)g.nb);
  const int64_t banks = batch * heads;
  const int64_t need = recap_pool_select_workspace_size(banks, g.nb, dim);
  REQUIRE(need > 0 && workspace_bytes >= need, "workspace of %lld bytes, need %lld",
          (long long)workspace_bytes, (long long)need);
  REQUIRE(aligned16(workspace), "workspace must be 16-byte aligned");
  // keep = max(1, round(density * nb)), Python's round-half-even (recap/sparse/attention.py:84)
  int64_t keep = (int64_t)std::nearbyint(density * (double)g.nb);
  keep = keep < 1 ? 1 : (keep > g.nb ? g.nb : keep);
  float* q_means = static_cast<float*>(workspace);
  float* scores = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                           align256(banks * g.nb * dim * 4));
  CHECK(recap_pool_blocks(q, dtype, batch, heads, dim, stride_b, stride_h, stride_n, rowmap,
                          n_tokens, n_video, q_means, stream));
  CHECK(recap_block_scores(q_means, k_means, banks, g.nb, dim, scale, scores, stream));
  CHECK(recap_topk_blocks(scores, banks, g.nb, keep, n_video % kBlock != 0 ? 1 : 0, partition,
                          stream));
  return recap_kernel_block_mask(partition, banks, n_tokens, n_video, kernel_mask, stream);
}

int recap_mask_overlap(const uint8_t* new_mask, const uint8_t* old_mask, int64_t count,
                       uint64_t* work, void* stream) {
  REQUIRE(new_mask && old_mask && work, "NULL pointer");
  REQUIRE(count >= 0, "negative count");
  return hip_status(run_mask_overlap(new_mask, old_mask, count,
                                     reinterpret_cast<unsigned long long*>(work), as_stream(stream)),
                    "mask_overlap launch");
}

int64_t recap_closure_groups(int64_t n_video, int64_t group) {
  if (n_video < 1 || group < 1) return -1;
  const int64_t nb = (n_video + kBlock - 1) / kBlock;
  return (nb + group - 1) / group;
}

int recap_closure_stats(const void* k_tiles, const void* vt_tiles, const float* k_means,
                        int dtype, const void* u_hi_t, const void* u_lo_t, int64_t banks,
                        int64_t dim, int64_t n_tokens, int64_t n_video, int64_t group,
                        int flags, float* variance, float* cvk_partial, float* scatter_partial,
                        void* stream) {
  CHECK(check_common(dtype, dim));
  CHECK(check_tokens(n_tokens, n_video));
  REQUIRE(banks >= 1 && group >= 1, "bad banks/group");
  REQUIRE(flags == RECAP_CLOSURE_ROT || flags == (RECAP_CLOSURE_CVK | RECAP_CLOSURE_SCATTER) ||
              flags == (RECAP_CLOSURE_ROT | RECAP_CLOSURE_CVK),
          "unsupported closure flag set %d", flags);
  REQUIRE(k_tiles && k_means && aligned16(k_tiles), "k_tiles/k_means");
  if (flags & RECAP_CLOSURE_ROT) REQUIRE(u_hi_t && u_lo_t && variance && aligned16(u_hi_t) && aligned16(u_lo_t), "ROT needs u_hi_t, u_lo_t, variance");
  if (flags & RECAP_CLOSURE_CVK) REQUIRE(vt_tiles && cvk_partial && aligned16(vt_tiles), "CVK needs vt_tiles, cvk_partial");
  if (flags & RECAP_CLOSURE_SCATTER) REQUIRE(scatter_partial != nullptr, "SCATTER needs scatter_partial");
  const Geom g = geometry(n_tokens, n_video);
  ClosureArgs a{};
  a.kp = static_cast<const uint16_t*>(k_tiles); a.vp = static_cast<const uint16_t*>(vt_tiles);
  a.kmean = k_means;
  a.u_hi_t = static_cast<const uint16_t*>(u_hi_t); a.u_lo_t = static_cast<const uint16_t*>(u_lo_t);
  a.banks = (int)banks; a.nb = (int)g.nb; a.tb = (int)g.tb; a.n_video = (int)n_video;
  a.group = (int)group; a.groups = (int)recap_closure_groups(n_video, group);
  a.var = variance; a.cvk_part = cvk_partial; a.scat_part = scatter_partial;
  return hip_status(run_closure(a, dtype, (int)dim, flags, as_stream(stream)), "closure launch");
}

int recap_partial_reduce(const float* partial, int64_t banks, int64_t groups, int64_t elems,
                         float divisor, float* out, void* stream) {
  REQUIRE(partial && out, "NULL pointer");
  REQUIRE(banks >= 1 && groups >= 1 && elems >= 1, "bad sizes");
  return hip_status(run_partial_reduce(partial, (int)banks, (int)groups, (int)elems, divisor, out,
                                       as_stream(stream)),
                    "partial_reduce launch");
}

int recap_symmetric_eigen(const float* a, int64_t batch, int64_t n, float* eigenvalues,
                          float* eigenvectors, void* stream) {
  REQUIRE(a && eigenvalues && eigenvectors, "NULL pointer");
  REQUIRE(batch >= 1 && batch <= 65535, "bad batch %lld", (long long)batch);
  REQUIRE(n >= 1 && n <= 128, "matrix order %lld outside [1, 128]", (long long)n);
  EigenArgs e{};
  e.a = a; e.batch = (int)batch; e.n = (int)n; e.m = (int)(n + (n & 1));
  e.max_sweeps = 40; e.values = eigenvalues; e.vectors = eigenvectors;
  return hip_status(run_symmetric_eigen(e, as_stream(stream)), "symmetric_eigen launch");
}

int recap_coarse_tables(const float* variance, const float* k_means, const float* v_means,
                        int dtype, int64_t banks, int64_t n_blocks, int64_t dim, int64_t rank,
                        void* w, void* kbar, void* vbar, void* stream) {
  CHECK(check_common(dtype, dim));
  REQUIRE(variance && k_means && v_means && w && kbar && vbar, "NULL pointer");
  REQUIRE(banks >= 1 && n_blocks >= 1 && rank >= 0, "bad sizes");
  TablesArgs a{variance, k_means, v_means, (int)banks, (int)n_blocks, (int)dim, (int)rank,
               static_cast<uint16_t*>(w), static_cast<uint16_t*>(kbar), static_cast<uint16_t*>(vbar)};
  return hip_status(run_tables(a, dtype, as_stream(stream)), "coarse_tables launch");
}

int64_t recap_coarse_w_width(int dtype, int64_t dim, int64_t rank) {
  if (check_common(dtype, dim) != RECAP_OK || rank < 0) return -1;
  return coarse_folded(dtype, (int)dim, (int)rank) ? kFoldCols : dim;
}

int recap_basis_tables(const float* basis, const float* cvk, int dtype, int64_t banks,
                       int64_t dim, void* u_hi_t, void* u_lo_t, void* u_t, void* cvk_t,
                       void* stream) {
  CHECK(check_common(dtype, dim));
  REQUIRE(basis != nullptr, "basis is NULL");
  REQUIRE(cvk_t == nullptr || cvk != nullptr, "cvk_t requested without cvk");
  REQUIRE(banks >= 1, "bad banks");
  BasisArgs a{basis, cvk, (int)banks, (int)dim, static_cast<uint16_t*>(u_hi_t),
              static_cast<uint16_t*>(u_lo_t), static_cast<uint16_t*>(u_t), static_cast<uint16_t*>(cvk_t)};
  return hip_status(run_basis_tables(a, dtype, as_stream(stream)), "basis_tables launch");
}

int recap_coarse_tail(const void* q, int dtype, int64_t batch, int64_t heads, int64_t dim,
                      int64_t stride_b, int64_t stride_h, int64_t stride_n,
                      const int32_t* rowmap, const uint8_t* partition, const void* kbar,
                      const void* vbar, const void* w, const void* u_t, const void* cvk_t,
                      int64_t n_tokens, int64_t n_video, float scale, float theta,
                      int64_t rank, const float* glref, void* go, float* gl,
                      float* drift_partial, void* stream) {
  CHECK(check_common(dtype, dim));
  CHECK(check_tokens(n_tokens, n_video));
  CHECK(check_qkv("q", q, batch, heads, stride_b, stride_h, stride_n));
  REQUIRE(rowmap && partition && kbar && vbar && w && u_t && cvk_t, "NULL pointer");
  REQUIRE(std::isfinite(scale) && scale > 0.0f, "scale must be positive and finite");
  REQUIRE(theta >= 0.0f, "theta must be non-negative");
  REQUIRE(rank >= 0 && rank <= dim, "rank %lld outside [0, dim]", (long long)rank);
  REQUIRE(aligned16(kbar) && aligned16(vbar) && aligned16(w) && aligned16(u_t) && aligned16(cvk_t),
          "tables must be 16-byte aligned");
  const Geom g = geometry(n_tokens, n_video);
  REQUIRE(g.nb <= 4096, "too many video blocks (%lld > 4096)", (long long)g.nb);
  // No full video block: no refined rows, nothing to write (go, gl may be empty buffers).
  if (g.rows == 0) return RECAP_OK;
  REQUIRE(go && gl && aligned16(go), "go and gl must be non-NULL, go 16-byte aligned");
  REQUIRE(glref == nullptr || drift_partial != nullptr, "glref needs drift_partial");
  CoarseArgs a{};
  a.q = static_cast<const uint16_t*>(q); a.sB = stride_b; a.sH = stride_h; a.sN = stride_n;
  a.rowmap = rowmap; a.partition = partition;
  a.kbar = static_cast<const uint16_t*>(kbar); a.vbar = static_cast<const uint16_t*>(vbar);
  a.w = static_cast<const uint16_t*>(w);
  a.u_t = static_cast<const uint16_t*>(u_t); a.cvk = static_cast<const uint16_t*>(cvk_t);
  a.heads = (int)heads; a.banks = (int)(batch * heads); a.nb = (int)g.nb;
  a.n_video = (int)n_video; a.rows = (int)g.rows; a.qtiles = (int)(g.rows / kBlock);
  a.scale = scale; a.theta = theta; a.rank = (int)rank; a.glref = glref;
  a.go = static_cast<uint16_t*>(go); a.gl = gl; a.drift_part = drift_partial;
  return hip_status(run_coarse(a, dtype, (int)dim, as_stream(stream)), "coarse_tail launch");
}

int recap_drift_center(const float* drift_partial, int64_t banks, int64_t n_video, float* center,
                       void* stream) {
  REQUIRE(center, "NULL pointer");
  REQUIRE(banks >= 1 && n_video >= 1, "bad banks/n_video");
  const int64_t rows = (n_video / kBlock) * kBlock;
  if (rows == 0) return RECAP_OK;  // no refined rows: no centre is used
  REQUIRE(drift_partial, "NULL pointer");
  return hip_status(run_drift_center(drift_partial, (int)banks, (int)(rows / kBlock), (int)rows, center,
                                     as_stream(stream)),
                    "drift_center launch");
}

static int attn_common(const void* q, int dtype, int64_t batch, int64_t heads, int64_t dim,
                       int64_t sb, int64_t sh, int64_t sn, const void* k_tiles,
                       const void* vt_tiles, const int32_t* rowmap, int64_t n_tokens,
                       int64_t n_video, AttnArgs& a) {
  CHECK(check_common(dtype, dim));
  CHECK(check_tokens(n_tokens, n_video));
  CHECK(check_qkv("q", q, batch, heads, sb, sh, sn));
  REQUIRE(k_tiles && vt_tiles && rowmap, "NULL tiles or rowmap");
  REQUIRE(aligned16(k_tiles) && aligned16(vt_tiles), "tiles must be 16-byte aligned");
  const Geom g = geometry(n_tokens, n_video);
  REQUIRE(g.tb <= 2048, "too many kernel blocks (%lld > 2048)", (long long)g.tb);
  a.q = static_cast<const uint16_t*>(q); a.qsB = sb; a.qsH = sh; a.qsN = sn;
  a.kp = static_cast<const uint16_t*>(k_tiles); a.vp = static_cast<const uint16_t*>(vt_tiles);
  a.rowmap = rowmap;
  a.heads = (int)heads; a.banks = (int)(batch * heads);
  a.n_tokens = (int)n_tokens; a.tb = (int)g.tb;
  // Long rows, started first: the text rows (from ds) and a ragged last video block, which
  // the selection keeps dense (recap/sparse/attention.py:88-94).
  a.ds = (int)((n_video % kBlock) != 0 ? g.nb - 1 : g.ds);
  a.rows = (int)g.rows;
  return RECAP_OK;
}

int recap_block_sparse_attn(const void* q, int dtype, int64_t batch, int64_t heads,
                            int64_t dim, int64_t stride_b, int64_t stride_h, int64_t stride_n,
                            const void* k_tiles, const void* vt_tiles, const int32_t* rowmap,
                            const uint8_t* kernel_mask, int64_t n_tokens, float scale,
                            void* head_out, float* head_lse, void* stream) {
  AttnArgs a{};
  // The head branch does not use the video/text split; any n_video <= n_tokens works.
  CHECK(attn_common(q, dtype, batch, heads, dim, stride_b, stride_h, stride_n, k_tiles, vt_tiles,
                    rowmap, n_tokens, n_tokens, a));
  REQUIRE(kernel_mask && head_out && head_lse, "NULL mask or output");
  REQUIRE(aligned16(head_out), "head_out must be 16-byte aligned");
  a.kmask = kernel_mask; a.ds = a.tb;
  CHECK(set_scale(a, scale));
  a.head_out = static_cast<uint16_t*>(head_out); a.head_lse = head_lse;
  return hip_status(run_attention(a, dtype, (int)dim, kModeHead, as_stream(stream)), "attention launch");
}

int recap_dense_attn(const void* q, int dtype, int64_t batch, int64_t heads, int64_t dim,
                     int64_t stride_b, int64_t stride_h, int64_t stride_n, const void* k_tiles,
                     const void* vt_tiles, const int32_t* rowmap, int64_t n_tokens, float scale,
                     void* out, int64_t out_stride_b, int64_t out_stride_h,
                     int64_t out_stride_n, float* lse, void* stream) {
  AttnArgs a{};
  CHECK(attn_common(q, dtype, batch, heads, dim, stride_b, stride_h, stride_n, k_tiles, vt_tiles,
                    rowmap, n_tokens, n_tokens, a));
  CHECK(check_qkv("out", out, batch, heads, out_stride_b, out_stride_h, out_stride_n));
  REQUIRE(lse != nullptr, "lse is NULL");
  a.ds = a.tb;
  CHECK(set_scale(a, scale));
  a.out = static_cast<uint16_t*>(out); a.osB = out_stride_b; a.osH = out_stride_h; a.osN = out_stride_n;
  a.lse_native = lse;
  return hip_status(run_attention(a, dtype, (int)dim, kModeDense, as_stream(stream)), "attention launch");
}

int recap_dense_head_attn(const void* q, int dtype, int64_t batch, int64_t heads, int64_t dim,
                          int64_t stride_b, int64_t stride_h, int64_t stride_n,
                          const void* k_tiles, const void* vt_tiles, const int32_t* rowmap,
                          const uint8_t* kernel_mask, int64_t n_tokens, float scale, void* out,
                          int64_t out_stride_b, int64_t out_stride_h, int64_t out_stride_n,
                          float* lse, void* head_out, float* head_lse, uint32_t* work_queue,
                          void* stream) {
  AttnArgs a{};
  CHECK(attn_common(q, dtype, batch, heads, dim, stride_b, stride_h, stride_n, k_tiles, vt_tiles,
                    rowmap, n_tokens, n_tokens, a));
  CHECK(check_qkv("out", out, batch, heads, out_stride_b, out_stride_h, out_stride_n));
  REQUIRE(kernel_mask != nullptr, "kernel_mask is NULL");
  REQUIRE(lse != nullptr && head_out != nullptr && head_lse != nullptr, "lse/head_out/head_lse NULL");
  a.kmask = kernel_mask;
  a.ds = a.tb;  // every query block walks all tb blocks: no long items to start first
  CHECK(set_scale(a, scale));
  a.out = static_cast<uint16_t*>(out); a.osB = out_stride_b; a.osH = out_stride_h; a.osN = out_stride_n;
  a.lse_native = lse;
  a.head_out = static_cast<uint16_t*>(head_out); a.head_lse = head_lse;
  CHECK(set_queue(a, work_queue, as_stream(stream)));
  return hip_status(run_attention(a, dtype, (int)dim, kModeDenseHead, as_stream(stream)), "attention launch");
}

int recap_sparse_merge_attn(const void* q, int dtype, int64_t batch, int64_t heads,
                            int64_t dim, int64_t stride_b, int64_t stride_h, int64_t stride_n,
                            const void* k_tiles, const void* vt_tiles, const int32_t* rowmap,
                            const uint8_t* kernel_mask, int64_t n_tokens, int64_t n_video,
                            float scale, const void* go, const float* gl, const void* det,
                            const float* dl, const float* glref, const float* center,
                            float alpha_override, void* out, int64_t out_stride_b,
                            int64_t out_stride_h, int64_t out_stride_n, uint32_t* work_queue,
                            void* stream) {
  AttnArgs a{};
  CHECK(attn_common(q, dtype, batch, heads, dim, stride_b, stride_h, stride_n, k_tiles, vt_tiles,
                    rowmap, n_tokens, n_video, a));
  CHECK(check_qkv("out", out, batch, heads, out_stride_b, out_stride_h, out_stride_n));
  REQUIRE(kernel_mask != nullptr, "kernel_mask is NULL");
  if (a.rows > 0) {
    REQUIRE(go && gl && det && dl && aligned16(go) && aligned16(det), "merge inputs go/gl/det/dl");
    REQUIRE(alpha_override >= 0.0f || (glref && center), "drift weight needs glref and center");
  }
  a.kmask = kernel_mask;
  CHECK(set_scale(a, scale));
  a.out = static_cast<uint16_t*>(out); a.osB = out_stride_b; a.osH = out_stride_h; a.osN = out_stride_n;
  a.go = static_cast<const uint16_t*>(go); a.gl = gl; a.det = static_cast<const uint16_t*>(det);
  a.dl = dl; a.glref = glref; a.center = center;
  a.use_override = alpha_override >= 0.0f ? 1 : 0;
  a.alpha_override = alpha_override;
  CHECK(set_queue(a, work_queue, as_stream(stream)));
  return hip_status(run_attention(a, dtype, (int)dim, kModeMerge, as_stream(stream)), "attention launch");
}

int64_t recap_attn_queue_words(void) { return kQueueWords; }

int64_t recap_capture_partials(int64_t banks, int64_t dim, int64_t n_video) {
  if (banks < 1 || (dim != 64 && dim != 128) || n_video < 1) return -1;
  const int64_t rpb = 256 / (dim / 8);
  return banks * ((n_video / kBlock) * kBlock / rpb);
}

// With no refined rows (R = 0) a validation sums nothing: both sums are zero, written by a
// fill kernel (a caller may capture the call into a graph).  The R-sized glref is then an
// empty buffer, possibly NULL, so a non-NULL `stats` alone asks for the sums.
static int zero_stats(float* stats, hipStream_t s) {
  return hip_status(run_zero_words(reinterpret_cast<unsigned*>(stats), 2, s), "stats reset");
}

// Arguments of a refresh capture, validated; `work` is false when there is nothing to do
// (R = 0).
static int capture_args(const void* dense_out, int dtype, int64_t batch, int64_t heads,
                        int64_t dim, int64_t out_stride_b, int64_t out_stride_h,
                        int64_t out_stride_n, const float* dense_lse, const void* head_out,
                        const float* head_lse, const void* go, const float* gl,
                        const int32_t* rowmap, int64_t n_tokens, int64_t n_video, void* det,
                        float* dl, const float* glref, const float* center, float* stats,
                        CaptureArgs& a, bool& work) {
  CHECK(check_common(dtype, dim));
  CHECK(check_tokens(n_tokens, n_video));
  CHECK(check_qkv("dense_out", dense_out, batch, heads, out_stride_b, out_stride_h, out_stride_n));
  REQUIRE(dense_lse && head_out && head_lse && rowmap, "NULL pointer");
  REQUIRE(aligned16(head_out), "16-byte alignment");
  REQUIRE(glref == nullptr || stats, "validation needs stats");
  const Geom g = geometry(n_tokens, n_video);
  work = g.rows > 0;
  if (!work) return RECAP_OK;  // no refined rows: go, gl, det, dl may be empty buffers
  REQUIRE(go && gl && det && dl, "NULL pointer");
  REQUIRE(aligned16(go) && aligned16(det), "16-byte alignment");
  REQUIRE(glref == nullptr || center, "validation needs center");
  a.of = static_cast<const uint16_t*>(dense_out);
  a.osB = out_stride_b; a.osH = out_stride_h; a.osN = out_stride_n;
  a.lf = dense_lse; a.oh = static_cast<const uint16_t*>(head_out); a.lh = head_lse;
  a.go = static_cast<const uint16_t*>(go); a.gl = gl; a.rowmap = rowmap;
  a.heads = (int)heads; a.banks = (int)(batch * heads); a.n_tokens = (int)n_tokens;
  a.rows = (int)g.rows;
  a.det = static_cast<uint16_t*>(det); a.dl = dl;
  a.glref = glref; a.center = center;
  return RECAP_OK;
}

int recap_refresh_capture(const void* dense_out, int dtype, int64_t batch, int64_t heads,
                          int64_t dim, int64_t out_stride_b, int64_t out_stride_h,
                          int64_t out_stride_n, const float* dense_lse, const void* head_out,
                          const float* head_lse, const void* go, const float* gl,
                          const int32_t* rowmap, int64_t n_tokens, int64_t n_video, void* det,
                          float* dl, const float* glref, const float* center,
                          float* stat_partial, float* stats, void* stream) {
  CaptureArgs a{};
  bool work = false;
  CHECK(capture_args(dense_out, dtype, batch, heads, dim, out_stride_b, out_stride_h,
                     out_stride_n, dense_lse, head_out, head_lse, go, gl, rowmap, n_tokens,
                     n_video, det, dl, glref, center, stats, a, work));
  const bool validate = glref != nullptr;
  REQUIRE(!validate || stat_partial, "validation needs stat_partial");
  REQUIRE(!validate || (reinterpret_cast<uintptr_t>(stat_partial) & 7) == 0,
          "stat_partial must be 8-byte aligned");
  if (!work) return stats ? zero_stats(stats, as_stream(stream)) : RECAP_OK;
  a.stat_part = stat_partial;
  int blocks = 0;
  hipStream_t s = as_stream(stream);
  CHECK(hip_status(run_capture(a, dtype, (int)dim, &blocks, s), "capture launch"));
  if (validate) CHECK(hip_status(run_sum_pairs(stat_partial, a.banks * blocks, stats, s), "sum_pairs launch"));
  return RECAP_OK;
}

int recap_refresh_capture_noalloc(const void* dense_out, int dtype, int64_t batch,
                                  int64_t heads, int64_t dim, int64_t out_stride_b,
                                  int64_t out_stride_h, int64_t out_stride_n,
                                  const float* dense_lse, const void* head_out,
                                  const float* head_lse, const void* go, const float* gl,
                                  const int32_t* rowmap, int64_t n_tokens, int64_t n_video,
                                  void* det, float* dl, const float* glref,
                                  const float* center, float* stats, void* stream) {
  CaptureArgs a{};
  bool work = false;
  CHECK(capture_args(dense_out, dtype, batch, heads, dim, out_stride_b, out_stride_h,
                     out_stride_n, dense_lse, head_out, head_lse, go, gl, rowmap, n_tokens,
                     n_video, det, dl, glref, center, stats, a, work));
  const bool validate = glref != nullptr;
  if (validate) {
    const int64_t pairs = recap_capture_partials(batch * heads, dim, n_video);
    static_assert(kCaptureScratchPairs == RECAP_CAPTURE_NOALLOC_MAX_PAIRS, "scratch size");
    REQUIRE(pairs <= kCaptureScratchPairs,
            "validation needs %lld partial pairs; the static scratch holds %lld (4 MiB): use "
            "recap_refresh_capture with a caller workspace",
            (long long)pairs, (long long)kCaptureScratchPairs);
  }
  if (!work) return stats ? zero_stats(stats, as_stream(stream)) : RECAP_OK;
  float* scratch = nullptr;
  if (validate) CHECK(hip_status(capture_scratch_pointer(&scratch), "static scratch lookup"));
  a.stat_part = scratch;
  int blocks = 0;
  hipStream_t s = as_stream(stream);
  CHECK(hip_status(run_capture(a, dtype, (int)dim, &blocks, s), "capture launch"));
  if (validate) CHECK(hip_status(run_sum_pairs(scratch, a.banks * blocks, stats, s), "sum_pairs launch"));
  return RECAP_OK;
}

// Host-bank pager ------------------------------------------------------------------------

static Pager* as_pager(recap_pager* p) { return reinterpret_cast<Pager*>(p); }
static const Pager* as_pager(const recap_pager* p) { return reinterpret_cast<const Pager*>(p); }

static int check_slot_key(const Pager* p, int64_t key, int32_t slot) {
  REQUIRE(p != nullptr, "pager is NULL");
  REQUIRE(slot >= 0 && slot < pager_slots(p), "slot %d outside 0..%d", (int)slot,
          pager_slots(p) - 1);
  REQUIRE(key >= 0 && key < pager_keys(p), "key %lld outside 0..%lld", (long long)key,
          (long long)pager_keys(p) - 1);
  REQUIRE(pager_bound(p, slot), "slot %d has no bound device fields", (int)slot);
  return RECAP_OK;
}

int recap_pager_create(int64_t n_keys, int32_t n_slots, const int64_t* field_bytes,
                       int32_t n_fields, int32_t flags, recap_pager** out) {
  REQUIRE(out != nullptr && field_bytes != nullptr, "NULL pointer");
  REQUIRE(n_keys >= 1 && n_slots >= 1 && n_slots <= 8, "n_keys >= 1 and 1 <= n_slots <= 8");
  REQUIRE(n_fields >= 1 && n_fields <= 16, "1 <= n_fields <= 16");
  for (int32_t f = 0; f < n_fields; ++f)
    REQUIRE(field_bytes[f] >= 0, "field %d has a negative size", (int)f);
  REQUIRE((flags & ~RECAP_PAGER_TIMING) == 0, "unknown pager flags %d", (int)flags);
  Pager* p = nullptr;
  CHECK(hip_status(pager_create(n_keys, n_slots, field_bytes, n_fields,
                                (flags & RECAP_PAGER_TIMING) != 0, &p), "pager create"));
  *out = reinterpret_cast<recap_pager*>(p);
  return RECAP_OK;
}

int recap_pager_destroy(recap_pager* pager) {
  pager_destroy(as_pager(pager));
  return RECAP_OK;
}

int recap_pager_bind(recap_pager* pager, int32_t slot, void* const* device_fields) {
  Pager* p = as_pager(pager);
  REQUIRE(p != nullptr && device_fields != nullptr, "NULL pointer");
  REQUIRE(slot >= 0 && slot < pager_slots(p), "slot %d outside 0..%d", (int)slot,
          pager_slots(p) - 1);
  for (int f = 0; f < pager_fields(p); ++f)   // an empty field may have no memory
    REQUIRE(device_fields[f] != nullptr || pager_field_bytes(p, f) == 0,
            "device field %d is NULL", f);
  pager_bind(p, slot, device_fields);
  return RECAP_OK;
}

int recap_pager_reserve(recap_pager* pager, int64_t n_keys) {
  REQUIRE(pager != nullptr && n_keys >= 0, "bad arguments");
  return hip_status(pager_reserve(as_pager(pager), n_keys), "pinned host allocation");
}

int recap_pager_stage_in(recap_pager* pager, int64_t key, int32_t slot, void* stream) {
  CHECK(check_slot_key(as_pager(pager), key, slot));
  REQUIRE(pager_stored(as_pager(pager), key), "key %lld holds no bank yet", (long long)key);
  return hip_status(pager_stage_in(as_pager(pager), key, slot, as_stream(stream)), "stage_in");
}

int recap_pager_prefetch(recap_pager* pager, int64_t key, int32_t slot) {
  CHECK(check_slot_key(as_pager(pager), key, slot));
  if (!pager_stored(as_pager(pager), key)) return RECAP_OK;  // nothing to bring in yet
  return hip_status(pager_prefetch(as_pager(pager), key, slot), "prefetch");
}

int recap_pager_stage_out(recap_pager* pager, int64_t key, int32_t slot, void* stream) {
  CHECK(check_slot_key(as_pager(pager), key, slot));
  return hip_status(pager_stage_out(as_pager(pager), key, slot, as_stream(stream)), "stage_out");
}

int recap_pager_acquire(recap_pager* pager, int32_t slot, void* stream) {
  Pager* p = as_pager(pager);
  REQUIRE(p != nullptr && slot >= 0 && slot < pager_slots(p), "bad pager or slot");
  return hip_status(pager_acquire(p, slot, as_stream(stream)), "acquire");
}

int recap_pager_release(recap_pager* pager, int32_t slot, void* stream) {
  Pager* p = as_pager(pager);
  REQUIRE(p != nullptr && slot >= 0 && slot < pager_slots(p), "bad pager or slot");
  return hip_status(pager_release(p, slot, as_stream(stream)), "release");
}

int recap_pager_finish(recap_pager* pager) {
  REQUIRE(pager != nullptr, "pager is NULL");
  return hip_status(pager_finish(as_pager(pager)), "finish");
}

int recap_pager_stored(const recap_pager* pager, int64_t key) {
  const Pager* p = as_pager(pager);
  if (p == nullptr || key < 0 || key >= pager_keys(p)) return -1;
  return pager_stored(p, key) ? 1 : 0;
}

int64_t recap_pager_host_bytes(const recap_pager* pager) {
  return pager == nullptr ? -1 : pager_host_bytes(as_pager(pager));
}

int recap_pager_counts(const recap_pager* pager, int64_t* counts) {
  REQUIRE(pager != nullptr && counts != nullptr, "NULL pointer");
  pager_counts(as_pager(pager), counts);
  return RECAP_OK;
}

int recap_pager_copy_time(recap_pager* pager, double* total_ms, int64_t* copies) {
  REQUIRE(pager != nullptr && total_ms != nullptr && copies != nullptr, "NULL pointer");
  return hip_status(pager_copy_time(as_pager(pager), total_ms, copies), "copy timing");
}

int recap_pager_resize(recap_pager* pager, const int64_t* field_bytes, int32_t n_fields) {
  Pager* p = as_pager(pager);
  REQUIRE(p != nullptr && field_bytes != nullptr, "NULL pointer");
  REQUIRE(n_fields == pager_fields(p), "n_fields %d != the pager's %d fields", (int)n_fields,
          pager_fields(p));
  for (int32_t f = 0; f < n_fields; ++f)
    REQUIRE(field_bytes[f] >= 0, "field %d has a negative size", (int)f);
  return hip_status(pager_resize(p, field_bytes), "resize");
}

int recap_bank_copy_async(void* dst, const void* src, int64_t bytes, void* stream) {
  REQUIRE(dst && src, "NULL pointer");
  REQUIRE(bytes >= 0, "negative size");
  if (bytes == 0) return RECAP_OK;
  return hip_status(hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyDefault, as_stream(stream)),
                    "hipMemcpyAsync");
}

}  // extern "C"
