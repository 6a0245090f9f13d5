// Argument blocks and launchers of the corrected sparse-attention kernels.  The C ABI in
// abi.cpp validates the caller's arguments, fills these structs and calls run_*.
#pragma once

#include "common.hpp"

namespace recap {

// Fused reorder + pack + block pooling (pack_pool.hip).
struct PackPoolArgs {
  const uint16_t* x0; int64_t sB0, sH0, sN0;   // K (or Q when pooling only)
  const uint16_t* x1; int64_t sB1, sH1, sN1;   // V (pack mode)
  const int32_t* rowmap;                         // reordered row -> native token, [N]
  int heads, banks, n_tokens, n_video, nb, tb;
  uint16_t* kp; uint16_t* vp;                    // packed tiles [bank][tb][128*D]
  float* mean0; float* mean1;                    // fp32 block means [bank][nb][D]
};
hipError_t run_pack_pool(const PackPoolArgs& a, int dtype, int dim, bool pack, hipStream_t s);

// Block scores + top-k selection + kernel grid mask (select.hip).
struct ScoreArgs {
  const float* qm; const float* km; int banks, nb, dim; float scale; float* scores;
};
hipError_t run_block_scores(const ScoreArgs& a, hipStream_t s);
struct TopkArgs {
  const float* scores; int banks, nb, keep, force_last; uint8_t* partition;
};
hipError_t run_topk(const TopkArgs& a, hipStream_t s);
struct KmaskArgs {
  const uint8_t* partition; int banks, nb, tb, ds; uint8_t* kmask;
};
hipError_t run_kernel_mask(const KmaskArgs& a, hipStream_t s);
hipError_t run_mask_overlap(const uint8_t* a, const uint8_t* b, int64_t n, unsigned long long* out,
                            hipStream_t s);

// Closure statistics (closure.hip).
enum ClosureFlags { kRot = 1, kCvk = 2, kScatter = 4 };
struct ClosureArgs {
  const uint16_t* kp; const uint16_t* vp; const float* kmean;
  const uint16_t* u_hi_t; const uint16_t* u_lo_t;   // U^T as bf16 hi/lo pair [bank][D][D]
  int banks, nb, tb, n_video, group, groups;
  float* var;                                       // [bank][nb][D]
  float* cvk_part; float* scat_part;                // [bank][groups][D][D]
};
hipError_t run_closure(const ClosureArgs& a, int dtype, int dim, int flags, hipStream_t s);
hipError_t run_partial_reduce(const float* part, int banks, int groups, int elems, float divisor,
                              float* out, hipStream_t s);
struct TablesArgs {
  const float* var; const float* kmean; const float* vmean; int banks, nb, dim, rank;
  uint16_t* w_t; uint16_t* kbar_t; uint16_t* vbar_t;   // element type of the query
};

// Folded w table of the coarse tail.  fold_rank leaves w with r + 1 distinct values per
// block (the r leading variances, then one mean rho in every other column), so
// qsq.w = sum_{c<r} qsq_c w_c + rho * T with T = sum_{c>=r} qsq_c.  With T split into three
// bf16 parts (exact to fp32), that is a dot product over kFoldCols = 16 features
// [qsq_0 .. qsq_{r-1}, T_hi, T_mid, T_lo, 0 ...] . [w_0 .. w_{r-1}, rho, rho, rho, 0 ...]:
// one 32x32x16 MFMA per 32-block tile instead of dim / 16.  bf16 only (its exponent range
// holds T; fp16 could overflow), 1 <= r <= 13 and r < dim; otherwise the table keeps dim
// columns and the kernel its full dot product.
constexpr int kFoldCols = 16;
inline bool coarse_folded(int dtype, int dim, int rank) {
  return dtype == BF16::code && rank >= 1 && rank + 3 <= kFoldCols && rank < dim;
}
hipError_t run_tables(const TablesArgs& a, int dtype, hipStream_t s);
struct BasisArgs {
  const float* basis; const float* cvk; int banks, dim;
  uint16_t* u_hi_t; uint16_t* u_lo_t;    // bf16 split of U^T (closure statistics)
  uint16_t* u_t; uint16_t* cvk_t;        // U^T and C_vk in the query type (coarse tail)
};
hipError_t run_basis_tables(const BasisArgs& a, int dtype, hipStream_t s);

// Symmetric eigen-decomposition of the closure scatter (eigen.hip).
struct EigenArgs {
  const float* a; int batch, n, m, max_sweeps;   // m = n rounded up to even
  float* values; float* vectors;                 // [batch][n], [batch][n][n] (columns)
};
hipError_t run_symmetric_eigen(const EigenArgs& a, hipStream_t s);

// Coarse tail (coarse.hip).
struct CoarseArgs {
  const uint16_t* q; int64_t sB, sH, sN;
  const int32_t* rowmap; const uint8_t* partition;
  const uint16_t* kbar; const uint16_t* vbar; const uint16_t* w;   // [bank][nb][D]
  const uint16_t* u_t; const uint16_t* cvk;                        // [bank][D][D]
  int heads, banks, nb, n_video, rows, qtiles, rank;
  float scale, theta;
  const float* glref;                  // [bank][rows] or null
  uint16_t* go; float* gl;             // [bank][rows][D], [bank][rows]
  float* drift_part;                   // [bank][qtiles] (when glref)
};
hipError_t run_coarse(const CoarseArgs& a, int dtype, int dim, hipStream_t s);

// Block-sparse attention (attention.hip).
enum AttnMode { kModeHead = 0, kModeDense = 1, kModeMerge = 2, kModeDenseHead = 3 };
struct AttnArgs {
  const uint16_t* q; int64_t qsB, qsH, qsN;
  const uint16_t* kp; const uint16_t* vp;
  const int32_t* rowmap; const uint8_t* kmask;   // kmask null in dense mode
  int heads, banks, n_tokens, tb;
  int ds;                                        // first long (dense) query row, started first
  float scale_log2;
  uint16_t* head_out; float* head_lse;           // head / dense-head, reordered [bank][N](D),
                                                 // head_out in the query type
  uint16_t* out; int64_t osB, osH, osN;          // dense / dense-head / merge, native order
  float* lse_native;                             // dense / dense-head [bank][N]
  int rows; const uint16_t* go; const float* gl; const uint16_t* det; const float* dl;
  const float* glref; const float* center; float alpha_override; int use_override;
  unsigned* queue;   // kQueueWords zeroed words: per-XCD claim counters, or null (static)
};
hipError_t run_attention(const AttnArgs& a, int dtype, int dim, int mode, hipStream_t s);
// Claim counters of the attention launch's work queues: one per XCD, 128 bytes apart.
constexpr int kQueueStride = 32;
constexpr int kQueueWords = 8 * kQueueStride;
hipError_t run_zero_words(unsigned* p, int n, hipStream_t s);

// Refresh capture (capture.hip).
struct CaptureArgs {
  const uint16_t* of; int64_t osB, osH, osN;     // dense output, native order
  const float* lf;                               // dense LSE, native [bank][N]
  const uint16_t* oh; const float* lh;           // head branch (query type), reordered [bank][N](D)
  const uint16_t* go; const float* gl;           // coarse branch [bank][rows](D)
  const int32_t* rowmap;
  int heads, banks, n_tokens, rows;
  uint16_t* det; float* dl;                      // refinement (fp16 values), in place
  const float* glref; const float* center;       // validation inputs, null = no validation
  float* stat_part;                              // [bank][blocks][2]
};
hipError_t run_capture(const CaptureArgs& a, int dtype, int dim, int* blocks_per_bank,
                       hipStream_t s);
hipError_t run_sum_pairs(const float* part, int n, float* out2, hipStream_t s);
// Partial pairs of the allocation-free capture's static scratch (4 MiB per GPU), and its
// device address on the current device (looked up on the first call per device).
constexpr int64_t kCaptureScratchPairs = int64_t(1) << 19;
hipError_t capture_scratch_pointer(float** out);
hipError_t run_drift_center(const float* part, int banks, int tiles, int rows, float* center,
                            hipStream_t s);

// Host-bank pager (pager.hip): pinned host banks, device slots, prefetch and write-back
// streams.  Slot and key indices are checked by the caller (abi.hip).
struct Pager;
hipError_t pager_create(int64_t n_keys, int n_slots, const int64_t* field_bytes, int n_fields,
                        bool timing, Pager** out);
void pager_destroy(Pager* p);
int pager_slots(const Pager* p);
int64_t pager_keys(const Pager* p);
int pager_fields(const Pager* p);
int64_t pager_field_bytes(const Pager* p, int field);
bool pager_bound(const Pager* p, int slot);
bool pager_stored(const Pager* p, int64_t key);
int64_t pager_host_bytes(const Pager* p);
void pager_counts(const Pager* p, int64_t* out4);
void pager_bind(Pager* p, int slot, void* const* fields);
hipError_t pager_reserve(Pager* p, int64_t n_keys);
hipError_t pager_stage_in(Pager* p, int64_t key, int slot, hipStream_t s);
hipError_t pager_prefetch(Pager* p, int64_t key, int slot);
hipError_t pager_stage_out(Pager* p, int64_t key, int slot, hipStream_t s);
hipError_t pager_acquire(Pager* p, int slot, hipStream_t s);
hipError_t pager_release(Pager* p, int slot, hipStream_t s);
hipError_t pager_finish(Pager* p);
hipError_t pager_copy_time(Pager* p, double* total_ms, int64_t* n);
hipError_t pager_resize(Pager* p, const int64_t* field_bytes);

}  // namespace recap
