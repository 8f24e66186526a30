// MFMA fragment types and the lane layout of v_mfma_f32_32x32x16_bf16 (gfx950).
//
// For D[32x32] += A[32x16] * B[16x32] executed by one wave (lane l, g = l / 32):
//   A operand  lane l holds A[l % 32][8 g .. 8 g + 7]           (8 bf16)
//   B operand  lane l holds B[8 g .. 8 g + 7][l % 32]           (8 bf16)
//   D          lane l, register r holds D[8 (r / 4) + 4 g + (r % 4)][l % 32]
// i.e. a lane owns one column of the result.  The layout is checked on the GPU by
// tests/test_gpu_mfma_layout.py through edf_debug_mfma_32x32x16_bf16().
#pragma once

#include "edf_common.hpp"

namespace edf {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;

EDF_DEVICE f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

EDF_DEVICE bf16x8 cat4(bf16x4 lo, bf16x4 hi) {
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

EDF_DEVICE f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

// Row (within the 32-row tile) held by register r of a lane in half g.
EDF_DEVICE constexpr int d_row(int r, int g) { return 8 * (r >> 2) + 4 * g + (r & 3); }

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(4))) unsigned u32x4;

EDF_DEVICE unsigned pack_bf16x2(float lo, float hi) {
  bf16x2 v;
  v[0] = (bf16)lo;
  v[1] = (bf16)hi;
  return __builtin_bit_cast(unsigned, v);
}

// An accumulator tile X (column = lane % 32) reused as an MFMA operand that contracts
// over X's rows: the B fragment of X (B[k][j] = X[k][j]) and the A fragment of X^T are
// the same 8 values, rows 16 m + 8 g .. 16 m + 7 + 8 g of column lane % 32.  Registers
// 8m..8m+3 of half g hold rows 16m + 4g + 0..3 and registers 8m+4..8m+7 hold rows
// 16m + 8 + 4g + 0..3, so one v_permlane32_swap per register pair (lanes 32..63 of the
// first operand trade places with lanes 0..31 of the second) completes the fragment.
// m is 0 or 1 and must be a compile-time constant after unrolling.
EDF_DEVICE bf16x8 acc_kfrag(const f32x16& x, int m) {
  const unsigned a0 = pack_bf16x2(x[8 * m + 0], x[8 * m + 1]);
  const unsigned a1 = pack_bf16x2(x[8 * m + 2], x[8 * m + 3]);
  const unsigned b0 = pack_bf16x2(x[8 * m + 4], x[8 * m + 5]);
  const unsigned b1 = pack_bf16x2(x[8 * m + 6], x[8 * m + 7]);
  const auto s0 = __builtin_amdgcn_permlane32_swap(a0, b0, false, false);
  const auto s1 = __builtin_amdgcn_permlane32_swap(a1, b1, false, false);
  const u32x4 r = {s0[0], s1[0], s0[1], s1[1]};
  return __builtin_bit_cast(bf16x8, r);
}

// Store an accumulator tile with its rows contiguous: dst[lane%32 * ld + row] (bf16),
// four consecutive rows per 8-byte store; dst points at (row 0, column 0).
EDF_DEVICE void store_rows(bf16* dst, long ld, const f32x16& x, int li, int g, float scale = 1.0f) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    bf16x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = (bf16)(x[4 * q + e] * scale);
    *(bf16x4*)(dst + (long)li * ld + 8 * q + 4 * g) = v;
  }
}

// ds_read_b64_tr_b16 (gfx950): within each group of 16 lanes, with lane i supplying the
// address A_i of four consecutive bf16, lane j = 4 a + b receives element b of
// A_{a}, A_{a+4}, A_{a+8}, A_{a+12} (layout checked on the GPU by
// tests/test_gpu_mfma_layout.py).  Pointing lane i at row r0 + i / 4, column
// c0 + 4 (i % 4) of a row-major tile hands lane j the column c0 + j of rows r0..r0+3:
// a transposed operand straight from a row-major LDS tile.
EDF_DEVICE bf16x4 lds_read_tr16(const bf16* p) {
  typedef __attribute__((ext_vector_type(4))) short s16x4;
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p);
  return __builtin_bit_cast(bf16x4, v);
}

// LDS layout of a row-major bf16 tile with HD columns.  The LDS of gfx950 serves 64
// four-byte banks per cycle (measured with SQ_LDS_BANK_CONFLICT); MFMA row-operand reads
// take 16 bytes from each of 16 consecutive rows, transposed reads 8 bytes per lane from
// 4 consecutive rows x 64 bytes (32 lanes per cycle).  No row padding serves both, so for
// HD = 128 the rows are unpadded (256 bytes) and the 16-byte chunk c of row r is stored at
// c ^ h(r), h(r) = 4 (r % 4) + (r / 4) % 4: h is a bijection over any 16 consecutive
// rows, and 4 consecutive rows x 4 chunks land on 16 distinct chunk slots.  Other head
// sizes (parity paths) use rows padded by 16 bytes.  col must be a multiple of 4.
template <int HD>
EDF_DEVICE int lds_off(int row, int col) {
  if constexpr (HD == 128) {
    const int h = ((row & 3) << 2) | ((row >> 2) & 3);
    return row * 128 + (((col >> 3) ^ h) << 3) + (col & 7);
  } else {
    return row * (HD + 8) + col;
  }
}
template <int HD>
constexpr int lds_tile_elems(int rows) {
  return HD == 128 ? rows * 128 : rows * (HD + 8);
}

// ---- direct global->LDS tiles (head_dim 128 attention kernels) ------------------------
typedef __attribute__((address_space(3))) void lds_void;

// One 16-byte load per lane straight into LDS: lane l of the wave writes bytes
// [16 l, 16 l + 16) after the wave-uniform address lds.
EDF_DEVICE void dma16(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds(src, (lds_void*)lds, 16, 0, 0);
}

// LDS tile of R rows x 128 bf16 columns (R a multiple of 16) in blocks of 64 16-byte slots:
// block half * R / 8 + b8 holds rows 8 b8 .. 8 b8 + 7, chunks (of 8 columns) 8 half .. +7,
// chunk c' and row r' of the block in slot (c' ^ (b8 % 2)) * 8 + (r' ^ 4 ((c' / 2) % 2)).
// One DMA load fills one block from 8 half rows (8 cache lines); MFMA row operands (16 rows
// of one chunk per 16 lanes) and transposed reads (4 rows x 4 chunks x 8 bytes per 32
// lanes) each touch all 64 banks once; and every fragment address is one of two per-lane
// bases plus an immediate (the row-major XOR swizzle needs an address register per
// fragment, a column-major tile makes each DMA load touch 64 lines).
//
// Rows r0 .. r0 + R - 1 of a row-major [T][128] bf16 head into such a tile, through the
// buffer resource r of the head (T * 256 bytes): rows past the end read as zeros.  The
// workgroup's 4 waves issue R / 16 loads each, load j filling block j; a lane's byte offset
// within the tile is loop-invariant and the tile's row offset is a scalar.
template <int R>
EDF_DEVICE void stage_hb(rsrc_t r, bf16* dst, int r0, int wu, int l) {
  constexpr int IPW = R / 16;  // loads per wave
  static_assert(R % 16 == 0, "whole 8-row blocks for 4 waves");
#pragma unroll
  for (int i = 0; i < IPW; ++i) {
    const int j = wu * IPW + i;
    const int half = j / (R / 8), b8 = j % (R / 8);
    const int cp = (l >> 3) ^ (b8 & 1);
    const int rp = (l & 7) ^ (4 * ((cp >> 1) & 1));
    const unsigned off = (unsigned)(((8 * b8 + rp) * 128 + (8 * half + cp) * 8) * 2);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(dst + 512 * j), 16, off, r0 * 256, 0, 0);
  }
}

// Element offsets into such a tile.  Row operand (lane li, half g reads row rb + li, chunk
// 2 kk + g; rb a multiple of 32): hb_row_base(li, g, kk % 2) + hb_row_off<R>(kk, rb).
EDF_DEVICE int hb_row_base(int li, int g, int parity) {
  return ((li >> 3) * 64 + 8 * (g ^ ((li >> 3) & 1)) + ((li & 7) ^ (4 * parity))) << 3;
}
template <int R>
EDF_DEVICE constexpr int hb_row_off(int kk, int rb) {
  return ((kk >> 2) * (R / 8) * 64 + 16 * (kk & 3) + (rb / 8) * 64) << 3;
}
// Transposed read of rows rb + 16 kc + kr + 8 h, columns 32 dt + d0 .. + 3 (rb a multiple
// of 32, kr < 8, d0 a multiple of 4 below 32): hb_tr_base(kr, d0, h) + hb_tr_off<R>(dt, kc, rb).
EDF_DEVICE int hb_tr_base(int kr, int d0, int h) {
  const int cq = d0 >> 3;
  return ((h * 64 + (cq ^ h) * 8 + (kr ^ (4 * ((cq >> 1) & 1)))) << 3) + (d0 & 7);
}
template <int R>
EDF_DEVICE constexpr int hb_tr_off(int dt, int kc, int rb) {
  return ((dt >> 1) * (R / 8) * 64 + (rb / 8 + 2 * kc) * 64 + 32 * (dt & 1)) << 3;
}

// vmcnt(0) only: the DMA loads and the plain loads of this wave have landed.
EDF_DEVICE void wait_vm() { __builtin_amdgcn_s_waitcnt(0x0F70); }

}  // namespace edf
