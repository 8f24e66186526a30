// Head layout changes around the fused attention kernels: the attention block's projection
// [B, T, P H d] (P stacked parts, e.g. q | k | v, each H heads of d) to P tensors [B, H, T, d]
// (the flash kernels' layout), and the way back, which is also the split's backward.  In the
// reference these are Nx reshapes / transposes around the fused attention call
// (lib/edifice/blocks/transformer_block.ex:118, multi_head_attention's head split), block glue.
//   split:  out_p[b, h, t, i] = x[b, t, p H d + h d + i]
//   merge:  y[b, t, p H d + h d + i] = in_p[b, h, t, i]
// One pass each, 16-byte accesses when d and the pointers allow (one element per thread
// otherwise); one workgroup row per (b, t), consecutive threads walk d within a head row on
// both sides.
#include <stdint.h>

#include <algorithm>
#include <type_traits>

#include "edf_abi.hpp"
#include "edf_common.hpp"

namespace edf {
namespace {

constexpr int HD_NT = 256;
constexpr int HD_MAX_PARTS = 4;

struct HeadsArgs {
  char* part[HD_MAX_PARTS];  // the P tensors [B, H, T, d]
  char* flat;                // [B, T, P H d]
  int T, P, H, du;           // du: units per head row
};

// one row (b, t) of the flat tensor per blockIdx.x, its P H du units over blockIdx.y and the
// threads; E: bytes per unit (16, or the element size); MERGE: parts -> flat, else the reverse
template <int E, bool MERGE>
__global__ __launch_bounds__(HD_NT) void heads_kernel(HeadsArgs a) {
  using U = std::conditional_t<E == 16, uint4, std::conditional_t<E == 4, unsigned, unsigned short>>;
  const unsigned bt = blockIdx.x;
  const int hu = a.H * a.du;
  const int r = blockIdx.y * HD_NT + threadIdx.x;
  if (r >= a.P * hu) return;
  const int p = r / hu, r2 = r - p * hu, h = r2 / a.du, i = r2 - h * a.du;
  const unsigned b = bt / (unsigned)a.T, t = bt - b * (unsigned)a.T;
  char* base = p == 0 ? a.part[0] : p == 1 ? a.part[1] : p == 2 ? a.part[2] : a.part[3];
  U* pp = reinterpret_cast<U*>(base) + (((long)b * a.H + h) * a.T + t) * a.du + i;
  U* fp = reinterpret_cast<U*>(a.flat) + (long)bt * a.P * hu + r;
  if constexpr (MERGE)
    *fp = *pp;
  else
    *pp = *fp;
}

int heads_run(hipStream_t s, bool merge, const void* const* parts, const void* flat, long B, long T, int P, int H,
              int d, int dtype) {
  const int es = dtype == EDF_BF16 ? 2 : 4;
  uintptr_t ptrs = (uintptr_t)flat;
  HeadsArgs a{};
  for (int p = 0; p < P; ++p) {
    a.part[p] = (char*)parts[p];
    ptrs |= (uintptr_t)parts[p];
  }
  a.flat = (char*)flat;
  a.T = (int)T, a.P = P, a.H = H;
  const bool vec = ((long)d * es) % 16 == 0 && !(ptrs & 15);
  a.du = vec ? (int)((long)d * es / 16) : d;
  const dim3 grid((unsigned)(B * T), (unsigned)((P * H * a.du + HD_NT - 1) / HD_NT));
  if (vec) {
    if (merge)
      heads_kernel<16, true><<<grid, HD_NT, 0, s>>>(a);
    else
      heads_kernel<16, false><<<grid, HD_NT, 0, s>>>(a);
  } else if (es == 2) {
    if (merge)
      heads_kernel<2, true><<<grid, HD_NT, 0, s>>>(a);
    else
      heads_kernel<2, false><<<grid, HD_NT, 0, s>>>(a);
  } else {
    if (merge)
      heads_kernel<4, true><<<grid, HD_NT, 0, s>>>(a);
    else
      heads_kernel<4, false><<<grid, HD_NT, 0, s>>>(a);
  }
  return check_launch(merge ? "head merge" : "head split");
}

int heads_check(const void* const* parts, const void* flat, long B, long T, int P, int H, int d, int dtype) {
  EDF_REQUIRE(B > 0 && T > 0 && H > 0 && d > 0, EDF_ERR_INVALID_ARG, "dimensions must be positive");
  EDF_REQUIRE(B * T < (1L << 31) && (long)P * H * d < (1L << 31), EDF_ERR_UNSUPPORTED,
              "B T and P H d must be below 2^31");
  EDF_REQUIRE(P >= 1 && P <= HD_MAX_PARTS, EDF_ERR_INVALID_ARG, "1 to %d parts", HD_MAX_PARTS);
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(parts && flat, EDF_ERR_INVALID_ARG, "null tensor pointer");
  for (int p = 0; p < P; ++p) EDF_REQUIRE(parts[p], EDF_ERR_INVALID_ARG, "null tensor pointer");
  return EDF_OK;
}

}  // namespace
}  // namespace edf

extern "C" {

int edf_heads_split(void* stream, const void* x, void* const* parts, long batch, long seq, int num_parts,
                    int num_heads, int head_dim, int dtype) {
  using namespace edf;
  int rc = heads_check((const void* const*)parts, x, batch, seq, num_parts, num_heads, head_dim, dtype);
  if (rc) return rc;
  return heads_run(as_stream(stream), false, (const void* const*)parts, x, batch, seq, num_parts, num_heads, head_dim,
                   dtype);
}

int edf_heads_merge(void* stream, const void* const* parts, void* y, long batch, long seq, int num_parts,
                    int num_heads, int head_dim, int dtype) {
  using namespace edf;
  int rc = heads_check(parts, y, batch, seq, num_parts, num_heads, head_dim, dtype);
  if (rc) return rc;
  return heads_run(as_stream(stream), true, parts, y, batch, seq, num_parts, num_heads, head_dim, dtype);
}

}  // extern "C"
