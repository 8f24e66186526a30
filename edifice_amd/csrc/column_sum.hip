// Column sums of a row-major matrix: the bias gradients of the block models' dense layers
// (db = sum over rows of dy; in the reference, the gradient of Axon.dense's bias, which XLA
// derives), block glue beside the layer norm and the loss.
//   out[c] = sum_r x[r, c]   (x [rows, cols] in dtype, out [cols] in out_dtype, f32 inside)
// Two stages, summed in a fixed order (deterministic, no atomics): each workgroup sums a
// slice of rows for 128 columns (a wave reads two adjacent elements per lane, the four waves
// of a workgroup take interleaved rows and are added in LDS), one float32 partial per slice;
// then four waves per 64 columns split the slices and are added in LDS (with a single slice
// the first stage writes the result).  Few rows (the float32 partials of a split product,
// summed and rounded once): one pass, each thread summing 16 bytes of adjacent columns over
// all rows in row order.
#include <stdint.h>

#include <algorithm>

#include "edf_abi.hpp"
#include "edf_common.hpp"

namespace edf {
namespace {

constexpr int CS_NT = 256;
constexpr int CS_CB = 128;        // columns per workgroup in stage 1 (two per lane)
constexpr int CS_SLICES = 64;     // row slices at most (stage 2 reads 16 partials per thread)
constexpr int CS_MIN_ROWS = 64;   // rows per slice at least
constexpr int CS_FEW_ROWS = 32;   // at most this many rows: the one-pass column-vector kernel
constexpr int CS_ROWS_WG = 8192;  // its workgroups at most (grid-stride beyond)

template <typename T> EDF_DEVICE void ld2(const T* p, float& a, float& b);
template <> EDF_DEVICE void ld2<bf16>(const bf16* p, float& a, float& b) {
  const unsigned u = *reinterpret_cast<const unsigned*>(p);
  a = __builtin_bit_cast(float, u << 16);
  b = __builtin_bit_cast(float, u & 0xffff0000u);
}
template <> EDF_DEVICE void ld2<float>(const float* p, float& a, float& b) {
  const float2 f = *reinterpret_cast<const float2*>(p);
  a = f.x;
  b = f.y;
}

// part [nslice][cols]: slice s covers rows [s * rps, (s + 1) * rps); PAIR: cols even and the
// rows 2-element aligned, so a lane reads two adjacent columns at once.  TO: with one slice
// (few rows, e.g. the partials of a split product) the sums go straight to the output type.
template <typename T, bool PAIR, typename TO = float>
__global__ __launch_bounds__(CS_NT) void cs_part_kernel(const T* __restrict__ x, TO* __restrict__ part, long rows,
                                                       int cols, long rps) {
  __shared__ float s_acc[4][CS_CB];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c0 = blockIdx.x * CS_CB + 2 * lane;
  const long r0 = (long)blockIdx.y * rps, r1 = std::min(rows, r0 + rps);
  float a0 = 0.0f, a1 = 0.0f;
  if (PAIR && c0 < cols) {
#pragma unroll 8
    for (long r = r0 + w; r < r1; r += 4) {
      float u, v;
      ld2(x + r * cols + c0, u, v);
      a0 += u;
      a1 += v;
    }
  } else if (!PAIR) {
    for (long r = r0 + w; r < r1; r += 4) {
      if (c0 < cols) a0 += to_f32(x[r * cols + c0]);
      if (c0 + 1 < cols) a1 += to_f32(x[r * cols + c0 + 1]);
    }
  }
  s_acc[w][2 * lane] = a0;
  s_acc[w][2 * lane + 1] = a1;
  __syncthreads();
  if (threadIdx.x < CS_CB) {
    const int c = blockIdx.x * CS_CB + threadIdx.x;
    const float v = ((s_acc[0][threadIdx.x] + s_acc[1][threadIdx.x]) + s_acc[2][threadIdx.x]) + s_acc[3][threadIdx.x];
    if (c < cols) part[(long)blockIdx.y * cols + c] = from_f32<TO>(v);
  }
}

// 16 bytes of T as f32 (VW = 16 / sizeof(T) values) and VW values stored as TO
template <typename T> struct CsVec;
template <> struct CsVec<float> {
  static constexpr int VW = 4;
  static EDF_DEVICE void ld(const float* p, float* a) {
    const float4 f = *reinterpret_cast<const float4*>(p);
    a[0] = f.x, a[1] = f.y, a[2] = f.z, a[3] = f.w;
  }
};
template <> struct CsVec<bf16> {
  static constexpr int VW = 8;
  static EDF_DEVICE void ld(const bf16* p, float* a) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const unsigned w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[2 * i] = __builtin_bit_cast(float, w4[i] << 16);
      a[2 * i + 1] = __builtin_bit_cast(float, w4[i] & 0xffff0000u);
    }
  }
};
template <typename TO, int VW> EDF_DEVICE void cs_stv(TO* p, const float* a) {
  if constexpr (sizeof(TO) == 4) {
#pragma unroll
    for (int j = 0; j < VW; j += 4)
      *reinterpret_cast<float4*>(p + j) = make_float4(a[j], a[j + 1], a[j + 2], a[j + 3]);
  } else {
    unsigned w[VW / 2];
#pragma unroll
    for (int i = 0; i < VW / 2; ++i)
      w[i] = (unsigned)__builtin_bit_cast(unsigned short, (bf16)a[2 * i]) |
             ((unsigned)__builtin_bit_cast(unsigned short, (bf16)a[2 * i + 1]) << 16);
    if constexpr (VW == 8)
      *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
    else
      *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
  }
}

// rows <= CS_FEW_ROWS, cols a multiple of VW, x and out 16-byte aligned: thread v sums columns
// [v VW, (v + 1) VW) over rows 0, 1, ... in order
template <typename T, typename TO>
__global__ __launch_bounds__(CS_NT) void cs_rows_kernel(const T* __restrict__ x, TO* __restrict__ out, int rows,
                                                       long cols) {
  constexpr int VW = CsVec<T>::VW;
  const long nvec = cols / VW;
  for (long v = (long)blockIdx.x * CS_NT + threadIdx.x; v < nvec; v += (long)gridDim.x * CS_NT) {
    float a[VW], b[VW];
#pragma unroll
    for (int i = 0; i < VW; ++i) a[i] = 0.0f;
#pragma unroll 8
    for (int r = 0; r < rows; ++r) {
      CsVec<T>::ld(x + r * cols + v * VW, b);
#pragma unroll
      for (int i = 0; i < VW; ++i) a[i] += b[i];
    }
    cs_stv<TO, VW>(out + v * VW, a);
  }
}

template <typename TO>
__global__ __launch_bounds__(CS_NT) void cs_final_kernel(const float* __restrict__ part, TO* __restrict__ out,
                                                        int nslice, int cols) {
  __shared__ float s_acc[4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  const int per = (nslice + 3) / 4, k0 = w * per, k1 = std::min(nslice, k0 + per);
  float a = 0.0f;
  if (c < cols) {
#pragma unroll 8
    for (int k = k0; k < k1; ++k) a += part[(long)k * cols + c];
  }
  s_acc[w][lane] = a;
  __syncthreads();
  if (w == 0 && c < cols) out[c] = from_f32<TO>(((s_acc[0][lane] + s_acc[1][lane]) + s_acc[2][lane]) + s_acc[3][lane]);
}

inline long cs_rows_per_slice(long rows, int /*cols*/) {
  return std::max((long)CS_MIN_ROWS, (rows + CS_SLICES - 1) / CS_SLICES);
}

template <typename T, typename TO>
int cs_run(hipStream_t s, const void* x, void* out, long rows, int cols, float* part) {
  constexpr int VW = CsVec<T>::VW;
  if (rows <= CS_FEW_ROWS && cols % VW == 0 && !(((uintptr_t)x | (uintptr_t)out) & 15)) {
    const long nvec = cols / VW;
    const unsigned grid = (unsigned)std::min((nvec + CS_NT - 1) / CS_NT, (long)CS_ROWS_WG);
    cs_rows_kernel<T, TO><<<grid, CS_NT, 0, s>>>((const T*)x, (TO*)out, (int)rows, cols);
    return check_launch("column sum (few rows)");
  }
  const long rps = cs_rows_per_slice(rows, cols);
  const int nslice = (int)((rows + rps - 1) / rps);
  const dim3 g1((cols + CS_CB - 1) / CS_CB, nslice);
  const bool pair = cols % 2 == 0 && ((uintptr_t)x & (2 * sizeof(T) - 1)) == 0;
  if (nslice == 1) {
    if (pair)
      cs_part_kernel<T, true, TO><<<g1, CS_NT, 0, s>>>((const T*)x, (TO*)out, rows, cols, rps);
    else
      cs_part_kernel<T, false, TO><<<g1, CS_NT, 0, s>>>((const T*)x, (TO*)out, rows, cols, rps);
    return check_launch("column sum");
  }
  if (pair)
    cs_part_kernel<T, true><<<g1, CS_NT, 0, s>>>((const T*)x, part, rows, cols, rps);
  else
    cs_part_kernel<T, false><<<g1, CS_NT, 0, s>>>((const T*)x, part, rows, cols, rps);
  int rc = check_launch("column sum");
  if (rc) return rc;
  cs_final_kernel<TO><<<(cols + 63) / 64, CS_NT, 0, s>>>(part, (TO*)out, nslice, cols);
  return check_launch("column sum (slices)");
}

}  // namespace
}  // namespace edf

extern "C" {

size_t edf_column_sum_workspace_bytes(long rows, int cols) {
  if (rows <= 0 || cols <= 0) return 0;
  const long rps = edf::cs_rows_per_slice(rows, cols);
  return (size_t)((rows + rps - 1) / rps) * cols * sizeof(float);
}

int edf_column_sum(void* stream, const void* x, void* out, void* workspace, size_t workspace_bytes, long rows,
                   int cols, int dtype, int out_dtype) {
  using namespace edf;
  EDF_REQUIRE(rows > 0 && cols > 0, EDF_ERR_INVALID_ARG, "dimensions must be positive");
  EDF_REQUIRE(valid_dtype(dtype) && valid_dtype(out_dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(x && out, EDF_ERR_INVALID_ARG, "null tensor pointer");
  const size_t need = edf_column_sum_workspace_bytes(rows, cols);
  EDF_REQUIRE(workspace && workspace_bytes >= need, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes", need);
  hipStream_t s = as_stream(stream);
  float* part = (float*)workspace;
  if (dtype == EDF_BF16)
    return out_dtype == EDF_BF16 ? cs_run<bf16, bf16>(s, x, out, rows, cols, part)
                                 : cs_run<bf16, float>(s, x, out, rows, cols, part);
  return out_dtype == EDF_BF16 ? cs_run<float, bf16>(s, x, out, rows, cols, part)
                               : cs_run<float, float>(s, x, out, rows, cols, part);
}

}  // extern "C"
