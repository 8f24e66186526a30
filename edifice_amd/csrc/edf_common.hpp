// Shared device helpers for the gfx950 kernels of edifice_amd.
//
// Storage types: every tensor is either IEEE float32 or bfloat16 (raw __bf16).
// Arithmetic is always float32 (bf16 is an I/O format only), matching the
// reference contract "bf16 I/O, f32 math" (native/cuda/precision.cuh:18-23).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

#define EDF_DEVICE __device__ __forceinline__

namespace edf {

typedef __bf16 bf16;

// ---- scalar load / store with conversion -----------------------------------
EDF_DEVICE float to_f32(float v) { return v; }
EDF_DEVICE float to_f32(bf16 v) { return (float)v; }

template <typename T> EDF_DEVICE T from_f32(float v);
template <> EDF_DEVICE float from_f32<float>(float v) { return v; }
template <> EDF_DEVICE bf16 from_f32<bf16>(float v) { return (bf16)v; }  // RNE

template <typename T> EDF_DEVICE float ld(const T* p, long i) { return to_f32(p[i]); }
template <typename T> EDF_DEVICE void st(T* p, long i, float v) { p[i] = from_f32<T>(v); }

// Branch-free guarded load: always reads p[ok ? i : safe] (an in-bounds element the
// caller names) and returns 0 when !ok.  Keeping loads out of divergent branches lets
// the compiler issue a whole block of them before the first wait.
template <typename T> EDF_DEVICE float ld_or0(const T* p, long i, bool ok, long safe = 0) {
  const float v = to_f32(p[ok ? i : safe]);
  return ok ? v : 0.0f;
}

// ---- raw buffer access ---------------------------------------------------------
// A raw buffer resource (V#) over [base, base + bytes), bytes < 2^31.  The hardware
// range-checks every access against it: a load at an offset >= bytes returns 0 and a
// store there is dropped, so kernels address padding lanes and steps with OOB_OFF
// instead of branching around the access.  The SGPR base plus a 32-bit VGPR offset
// also keeps 64-bit address arithmetic out of the vector registers.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr unsigned OOB_OFF = 0x80000000u;
constexpr int BUF_DWORD3 = 0x00020000;  // gfx9 raw buffer: 32-bit data format, no swizzle

EDF_DEVICE rsrc_t make_rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, BUF_DWORD3);
}

// storage-type bits of one element (T = float or bf16) and their conversions
template <typename T> struct Bits;
template <> struct Bits<float> { typedef unsigned type; };
template <> struct Bits<bf16> { typedef unsigned short type; };

template <typename T> EDF_DEVICE typename Bits<T>::type bload(rsrc_t r, unsigned off);
template <> EDF_DEVICE unsigned bload<float>(rsrc_t r, unsigned off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
template <> EDF_DEVICE unsigned short bload<bf16>(rsrc_t r, unsigned off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}
EDF_DEVICE float bits_f32(unsigned v) { return __builtin_bit_cast(float, v); }
EDF_DEVICE float bits_f32(unsigned short v) { return __builtin_bit_cast(float, (unsigned)v << 16); }

// AUX: the cache-policy immediate (BUF_NT marks a streaming store).  Two stores on the two
// sides of a lane-divergent branch that differ only in their resource are merged by the
// compiler into one store with a per-lane resource, which then runs once per distinct
// resource in the wave; a different AUX keeps them apart.
constexpr int BUF_NT = 2;
template <typename T, int AUX = 0> EDF_DEVICE void bstore(rsrc_t r, unsigned off, float v) {
  if constexpr (sizeof(T) == 4)
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, (int)off, 0, AUX);
  else
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, (bf16)v), r, (int)off, 0, AUX);
}

// Row stride (floats) of an LDS tile of 16 rows x dp columns that lanes write as (row =
// tid / 16, column = tid % 16 + 16 c): a ds_write_b32 resolves 32 lanes at a time over 32
// banks (word address mod 32), so the two rows of one half-wave sit 16 words apart mod 32;
// reads along a row stay contiguous.
constexpr int row16_stride(int dp) { return dp + (48 - dp % 32) % 32; }

// ---- math -------------------------------------------------------------------
constexpr float LOG2E = 1.4426950408889634f;

EDF_DEVICE float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
EDF_DEVICE float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// sigmoid(x) = 1 / (1 + 2^(-x log2 e)); exact reciprocal keeps f32 parity.
EDF_DEVICE float sigmoidf(float x) { return 1.0f / (1.0f + fast_exp2(-x * LOG2E)); }

// sigmoid with the hardware reciprocal (1 ulp) instead of an IEEE division: for gates on
// f32 math whose results are checked at 1e-4; 2^(-x log2 e) -> inf gives rcp(inf) = 0.
EDF_DEVICE float sigmoid_rcp(float x) { return fast_rcp(1.0f + fast_exp2(-x * LOG2E)); }

// softplus(x) = max(x, 0) + log1p(e^-|x|) from the hardware exp2 / log2: with t = e^-|x| in
// (0, 1], log2(1 + t) ln 2 for t >= 2^-10 (1 + t is exact to 2^-24), and t (1 - t / 2) below,
// whose error t^3 / 3 is under 2^-20 of the result
EDF_DEVICE float softplus_f(float x) {
  constexpr float LN2 = 0.6931471805599453f;
  const float t = fast_exp2(-fabsf(x) * LOG2E);
  const float lp = t < 0.0009765625f ? t * fmaf(-0.5f, t, 1.0f) : __builtin_amdgcn_logf(1.0f + t) * LN2;
  return fmaxf(x, 0.0f) + lp;
}

EDF_DEVICE float clampf(float x, float lo, float hi) { return fminf(fmaxf(x, lo), hi); }

// ---- compile-time loops ------------------------------------------------------
// static_for<N>(f) calls f(IC<0>{}), ..., f(IC<N-1>{}); inside f, decltype(i)::value is
// a constant expression (needed for instruction immediates such as DPP controls).
template <int J> struct IC { static constexpr int value = J; };
template <typename F, int... Is>
EDF_DEVICE void static_for_impl(std::integer_sequence<int, Is...>, F&& f) { (f(IC<Is>{}), ...); }
template <int N, typename F>
EDF_DEVICE void static_for(F&& f) { static_for_impl(std::make_integer_sequence<int, N>{}, f); }

// ---- cross-lane ----------------------------------------------------------------
// DPP row_newbcast:J (gfx90a and later): every lane receives lane J of its own 16-lane
// row.  With the same 16 values replicated in the four rows of a wave this is a
// wave-wide broadcast of value J, and the compiler folds it into the consuming VOP2
// instruction (v_mul_f32_dpp) when old = 0 and bound_ctrl is set.
template <int J>
EDF_DEVICE float row_bcast(float v) {
  static_assert(J >= 0 && J < 16, "lane within a row");
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x150 + J, 0xF, 0xF,
                                                               true));
}

// Sum over the 16 lanes of each DPP row, returned in every lane of the row: a rotation
// butterfly (row_ror 8, 4, 2, 1) of VALU DPP adds.  At each step a lane and its partner
// already hold equal values, so all 16 lanes end with the bitwise-same sum.
template <int CTRL>
EDF_DEVICE float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
EDF_DEVICE float row16_sum(float x) {
  x += dpp_f32<0x128>(x);  // row_ror:8
  x += dpp_f32<0x124>(x);  // row_ror:4
  x += dpp_f32<0x122>(x);  // row_ror:2
  x += dpp_f32<0x121>(x);  // row_ror:1
  return x;
}

// Lane swaps between the four 16-lane rows of a wave.  Inline assembly: the compiler's
// permlane swap builtins return the first register's new value in both halves of their
// result when the second half is read through __builtin_bit_cast.  The s_nop covers the
// wait states a VALU write needs before a permlane swap reads the register.
EDF_DEVICE void swap16(float& a, float& b) {  // odd rows of a <-> even rows of b
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
EDF_DEVICE void swap32(float& a, float& b) {  // rows 2, 3 of a <-> rows 0, 1 of b
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
// Reduce-scatter over the four rows: v[0..3] summed lane-wise over the rows, the lane in
// row r receiving the sum of v[rows4_item(r)] (rows4_item is its own inverse).
EDF_DEVICE constexpr int rows4_item(int r) { return 2 * (r & 1) + (r >> 1); }
EDF_DEVICE float rows4_scatter(float v0, float v1, float v2, float v3) {
  swap16(v0, v2);  // v0: rows 0, 2 keep v0, rows 1, 3 receive v2 of rows 0, 2
  swap16(v1, v3);
  float w0 = v0 + v2, w1 = v1 + v3;  // even rows: v0 / v1 of rows r, r + 1; odd rows: v2 / v3
  swap32(w0, w1);
  return w0 + w1;
}

// ---- launch-shape helpers -----------------------------------------------------
// MI355X dispatches consecutive workgroup ids round-robin over its 8 XCDs, each
// with a private L2.  remap_xcd() turns the hardware id into a logical id such
// that logical ids L, L+1, ... run on the same XCD, so neighbouring tiles that
// share cache lines also share an L2.  Identity when the grid is not a multiple
// of 8.
EDF_DEVICE int remap_xcd(int id, int total) {
  if ((total & 7) != 0) return id;
  const int per = total >> 3;
  return (id & 7) * per + (id >> 3);
}

// For a 2-D grid (x = block within a head, y = head): the (block, head) this workgroup
// takes, remapped with remap_xcd so that all blocks of a head run on one XCD and share
// its L2 (the K/V or Q/dO tiles every block of the head streams through).
EDF_DEVICE void head_block(int& blk, long& head) {
  const int nx = gridDim.x;
  const int logical = remap_xcd(blockIdx.x + nx * blockIdx.y, nx * gridDim.y);
  blk = logical % nx;
  head = logical / nx;
}

}  // namespace edf
