// Shared device helpers for the gfx950 (CDNA4) kernels of the corrected sparse-attention
// path: element types, MFMA wrappers, 64-wide wave reductions and packed-tile layouts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace recap {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kBlock = 128;        // tokens per block (query and key)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------------------------------
// Element types: values are stored as raw 16-bit words; arithmetic is fp32.

struct BF16 {
  static constexpr int code = 2;
  __device__ static inline float to_f(uint16_t h) { return __uint_as_float((unsigned)h << 16); }
  __device__ static inline uint16_t from_f(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);  // round to nearest even
  }
  __device__ static inline f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

struct F16 {
  static constexpr int code = 1;
  __device__ static inline float to_f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
  }
  __device__ static inline uint16_t from_f(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
  }
  __device__ static inline f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

__device__ inline float bf16_to_f(uint16_t h) { return BF16::to_f(h); }
__device__ inline uint16_t f_to_bf16(float f) { return BF16::from_f(f); }
__device__ inline float f16_to_f(uint16_t h) { return F16::to_f(h); }
__device__ inline uint16_t f_to_f16(float f) { return F16::from_f(f); }

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Two fp32 values rounded to the 16-bit type and packed (lo in bits 0-15): one
// v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32 per pair.
template <class T>
__device__ inline unsigned pack2(float lo, float hi) {
  if constexpr (T::code == 2) {
    return __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
  } else {
    return __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{lo, hi}, f16x2));
  }
}

// Two fp32 values each rounded to the 16-bit type (to nearest even) and widened back: one
// conversion per pair.
template <class T>
__device__ inline void round2(float& lo, float& hi) {
  const unsigned u = pack2<T>(lo, hi);
  if constexpr (T::code == 2) {
    lo = __uint_as_float(u << 16);
    hi = __uint_as_float(u & 0xffff0000u);
  } else {
    lo = T::to_f((uint16_t)u);
    hi = T::to_f((uint16_t)(u >> 16));
  }
}

// ---------------------------------------------------------------------------------------
// 32x32 MFMA output layout (all v_mfma_f32_32x32x* ops): lane l, register r holds
// D[row = 8*(r/4) + 4*(l/32) + r%4][col = l%32].  A operand: lane l holds 8 consecutive
// k of row l%32, k-group l/32.  B operand: lane l holds 8 consecutive k of column l%32.
__device__ inline int mfma_row(int r, int g) { return 8 * (r >> 2) + 4 * g + (r & 3); }

// Swap bits 2 and 3 of a position: maps an MFMA k-slot (8*g + e within a 16-group) to
// the output row (8*(e/4) + 4*g + e%4) that held it, so a 32x32 result can feed the
// next MFMA as its B operand without a register shuffle.
__host__ __device__ inline int swap23(int p) {
  return (p & ~12) | ((p & 4) << 1) | ((p & 8) >> 1);
}

// ---------------------------------------------------------------------------------------
// Lane pairs (l, l^32) hold the two halves of one 32x32 output column.

__device__ inline float pair_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __builtin_elementwise_maximum(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ inline float pair_sum(float x) {
  // Both lanes compute low-half + high-half in the same order.
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Fixed-order sum over lanes 0..31 of a wave (butterfly), result in every lane.
__device__ inline float half_wave_sum(float x) {
  for (int off = 16; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

__device__ inline float wave_sum(float x) {
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// ---------------------------------------------------------------------------------------
// Work-item order: blockIdx -> linear item so that each XCD (8 per MI355X, workgroups
// dealt round-robin) gets a contiguous range of items and hence of banks, keeping one
// bank's K/V tiles in that XCD's L2.
__device__ inline int xcd_linear(int bid, int n) {
  const int xcd = bid & 7, slot = bid >> 3;
  const int per = n >> 3, rem = n & 7;
  return xcd * per + min(xcd, rem) + slot;
}

// Work-item order for kernels whose items share data with their neighbours: items go to
// the XCDs in runs of `run` consecutive items (run 0 to XCD 0, run 1 to XCD 1, ...), so the
// items in flight on one XCD are neighbours (shared tiles stay in that XCD's L2) while all
// XCDs together stay within 8 * run consecutive items (one working set in the Infinity
// Cache).  The items left after the last full round of 8 runs are dealt round-robin.  The
// map is a bijection of [0, n).
__host__ __device__ inline int xcd_runs(int bid, int n, int run) {
  const int round = 8 * run;
  const int full = n / round * round;
  if (bid >= full) return bid;  // round-robin tail: identity keeps XCD i % 8
  const int xcd = bid & 7, slot = bid >> 3;
  return (slot / run * 8 + xcd) * run + slot % run;
}

// Packed tile geometry.  A K tile is [128 keys][D] with its 16-byte chunks XOR-swizzled by
// key row.  A V^T tile is two halves (keys 0-63, 64-127), each [D][64 positions] with
// 128-byte rows whose chunks are swizzled by d row; position p of the tile holds key
// swap23(p).  Keys 64h.. of K and half h of V^T are each one contiguous block, so a 64-key
// sub-tile is two contiguous images the attention kernel copies verbatim into LDS.
template <int D>
struct TileGeom {
  static constexpr int kRowBytes = D * 2;           // K tile row
  static constexpr int kChunks = D / 8;             // 16-byte chunks per K row
  static constexpr int kTileElems = kBlock * D;     // elements per K (or V^T) tile
  static constexpr int kTileBytes = kTileElems * 2;
  static constexpr int kHalfBytes = kTileBytes / 2; // one 64-key half of K or of V^T
  __host__ __device__ static inline int k_off(int key, int chunk) {  // bytes
    return key * kRowBytes + ((chunk ^ swz(key, kChunks)) << 4);
  }
  // chunk c (0..15) of V^T row d: positions 8c..8c+7
  __host__ __device__ static inline int vt_off(int d, int c) {  // bytes
    return (c >> 3) * kHalfBytes + d * 128 + (((c & 7) ^ swz(d, 8)) << 4);
  }
  // XOR pattern for rows of `chunks` 16-byte chunks: any 16 consecutive rows read at one
  // logical chunk land on distinct banks whether LDS serves 8 lanes x 16 B over 32 banks or
  // 16 lanes over 64 banks per cycle.  With 8-chunk (128-byte) rows, rows r and r+8 share
  // the bank half of r's parity, so bit 3 of the row flips the lowest chunk bit.
  __host__ __device__ static inline int swz(int row, int chunks) {
    return chunks == 16 ? (row & 15) : ((row & 7) ^ ((row >> 3) & 1));
  }
};

// LDS address space, for the buffer-load-to-LDS builtin's destination.
typedef __attribute__((address_space(3))) void lds_void;

// Word 3 of a raw buffer resource on CDNA (32-bit data format, no swizzle).
constexpr int kBufferRsrcWord3 = 0x00020000;

// Coarse-tail tables: one row per key block, and 32 blocks (slots) per tile of the coarse
// kernel, which gathers the rows of a tile into K-tile images (TileGeom<D>::k_off with the
// slot as the row).
constexpr int kCoarseSlots = 32;

// Four 16-bit elements in LDS, the operand of the transposing LDS read.
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 s16x4_lds;

__device__ inline u32x4 lds_load16(const char* base, int off) {
  return *reinterpret_cast<const u32x4*>(base + off);
}

}  // namespace recap
