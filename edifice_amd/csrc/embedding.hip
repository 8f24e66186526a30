// Token-embedding weight gradient: the input layer of the language models built on the fused
// blocks (Axon.embedding, e.g. lib/edifice/generative/show_o.ex:123; the hybrid decoder's
// token embedding), block glue in front of the first norm.
//   dW[v, :] = sum over positions p with ids[p] == v, in ascending p, of grad[p, :]
// (f32 sums rounded once; 0 for rows no position names and for padding_idx).
// Deterministic, no atomics: the (id, position) pairs are ordered by id with rocPRIM's stable
// radix sort (positions stay ascending within an id), one thread per vocabulary row finds
// where its run of the sorted ids starts (binary search), and one wave per row sums the run's
// gradient rows in order, with 16-byte loads when the row allows.  Every row of dW is written
// (the zero rows too), so no separate fill pass.
#include <stdint.h>

#include <algorithm>
#include <rocprim/device/device_radix_sort.hpp>

#include "edf_abi.hpp"
#include "edf_common.hpp"

namespace edf {
namespace {

constexpr int EB_NT = 256;  // four waves, one vocabulary row each

template <typename T> struct EbVec;
template <> struct EbVec<bf16> {
  static constexpr int W = 8;
  static EDF_DEVICE void add(const bf16* p, float* a) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const unsigned w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[2 * i] += __builtin_bit_cast(float, w4[i] << 16);
      a[2 * i + 1] += __builtin_bit_cast(float, w4[i] & 0xffff0000u);
    }
  }
  static EDF_DEVICE void st(bf16* p, const float* a) {
    unsigned w4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w4[i] = (unsigned)__builtin_bit_cast(unsigned short, (bf16)a[2 * i]) |
              ((unsigned)__builtin_bit_cast(unsigned short, (bf16)a[2 * i + 1]) << 16);
    *reinterpret_cast<uint4*>(p) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
  }
};
template <> struct EbVec<float> {
  static constexpr int W = 4;
  static EDF_DEVICE void add(const float* p, float* a) {
    const float4 f = *reinterpret_cast<const float4*>(p);
    a[0] += f.x, a[1] += f.y, a[2] += f.z, a[3] += f.w;
  }
  static EDF_DEVICE void st(float* p, const float* a) { *reinterpret_cast<float4*>(p) = make_float4(a[0], a[1], a[2], a[3]); }
};

// sort keys and values: key = id (ids outside [0, vocab) get key vocab, which no row reads;
// the forward lookup has already rejected them), value = position
__global__ __launch_bounds__(256) void eb_keys_kernel(const int64_t* __restrict__ ids, unsigned* __restrict__ keys,
                                                     int* __restrict__ pos, long n, long vocab) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t v = ids[i];
  keys[i] = (unsigned)((v < 0 || v >= vocab) ? vocab : v);
  pos[i] = (int)i;
}

// first index in sorted keys[0, n) whose key is >= v
EDF_DEVICE long lower_bound(const unsigned* __restrict__ keys, long n, unsigned v) {
  long lo = 0, hi = n;
  while (lo < hi) {
    const long mid = (lo + hi) >> 1;
    if (keys[mid] < v)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo;
}

// off[v] = start of row v's run in the sorted keys, v in [0, vocab] (off[vocab]: the end)
__global__ __launch_bounds__(256) void eb_offsets_kernel(const unsigned* __restrict__ keys, int* __restrict__ off,
                                                        long n, long vocab) {
  const long v = (long)blockIdx.x * 256 + threadIdx.x;
  if (v <= vocab) off[v] = (int)lower_bound(keys, n, (unsigned)v);
}

// one wave per row v of dW, its run [off[v], off[v + 1]); VEC: dim a multiple of W and the
// tensors 16-byte aligned
template <typename T, bool VEC>
__global__ __launch_bounds__(EB_NT) void eb_gather_kernel(const T* __restrict__ grad, const int* __restrict__ off,
                                                         const int* __restrict__ pos, T* __restrict__ dw, long vocab,
                                                         int dim, long padding_idx) {
  const int lane = threadIdx.x & 63;
  const long v = (long)blockIdx.x * (EB_NT / 64) + (threadIdx.x >> 6);
  if (v >= vocab) return;
  const long lo = off[v];
  const long hi = v == padding_idx ? lo : off[v + 1];
  T* out = dw + v * dim;
  if constexpr (VEC) {
    constexpr int W = EbVec<T>::W;
    for (int c0 = lane * W; c0 < dim; c0 += 64 * W) {
      float a[W];
#pragma unroll
      for (int i = 0; i < W; ++i) a[i] = 0.0f;
#pragma unroll 4
      for (long p = lo; p < hi; ++p) EbVec<T>::add(grad + (long)pos[p] * dim + c0, a);
      EbVec<T>::st(out + c0, a);
    }
  } else {
    for (int c = lane; c < dim; c += 64) {
      float a = 0.0f;
      for (long p = lo; p < hi; ++p) a += to_f32(grad[(long)pos[p] * dim + c]);
      out[c] = from_f32<T>(a);
    }
  }
}

inline size_t eb_align(size_t b) { return (b + 255) & ~(size_t)255; }

inline unsigned eb_bits(long vocab) {
  unsigned b = 1;
  while (b < 32 && (1ul << b) <= (unsigned long)vocab) ++b;  // keys run to vocab inclusive
  return b;
}

// rocPRIM's temporary storage for n pairs (0 on a query failure)
size_t eb_sort_bytes(long n, long vocab) {
  size_t bytes = 0;
  if (n <= 0) return 0;
  if (rocprim::radix_sort_pairs(nullptr, bytes, (unsigned*)nullptr, (unsigned*)nullptr, (int*)nullptr,
                                (int*)nullptr, (unsigned)n, 0u, eb_bits(vocab)) != hipSuccess)
    return 0;
  return bytes;
}

template <typename T>
int eb_run(hipStream_t s, const int64_t* ids, const void* grad, void* dw, char* ws, size_t sort_bytes, long n,
           long vocab, int dim, long padding_idx) {
  const size_t kb = eb_align((size_t)std::max(n, 1L) * 4);
  unsigned* keys_in = (unsigned*)ws;
  unsigned* keys = (unsigned*)(ws + kb);
  int* pos_in = (int*)(ws + 2 * kb);
  int* pos = (int*)(ws + 3 * kb);
  int* off = (int*)(ws + 4 * kb);
  void* tmp = ws + 4 * kb + eb_align((size_t)(vocab + 1) * 4);
  if (n > 0) {
    eb_keys_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(ids, keys_in, pos_in, n, vocab);
    int rc = check_launch("embedding backward keys");
    if (rc) return rc;
    size_t bytes = sort_bytes;
    const hipError_t e = rocprim::radix_sort_pairs(tmp, bytes, keys_in, keys, pos_in, pos, (unsigned)n, 0u,
                                                   eb_bits(vocab), s);
    EDF_REQUIRE(e == hipSuccess, EDF_ERR_LAUNCH, "embedding backward sort: %s", hipGetErrorString(e));
  }
  eb_offsets_kernel<<<(unsigned)((vocab + 1 + 255) / 256), 256, 0, s>>>(keys, off, n, vocab);
  int rc = check_launch("embedding backward offsets");
  if (rc) return rc;
  constexpr int W = EbVec<T>::W;
  const bool vec = dim % W == 0 && !(((uintptr_t)grad | (uintptr_t)dw) & 15);
  const unsigned grid = (unsigned)((vocab + EB_NT / 64 - 1) / (EB_NT / 64));
  if (vec)
    eb_gather_kernel<T, true><<<grid, EB_NT, 0, s>>>((const T*)grad, off, pos, (T*)dw, vocab, dim, padding_idx);
  else
    eb_gather_kernel<T, false><<<grid, EB_NT, 0, s>>>((const T*)grad, off, pos, (T*)dw, vocab, dim, padding_idx);
  return check_launch("embedding backward");
}

}  // namespace
}  // namespace edf

extern "C" {

size_t edf_embedding_backward_workspace_bytes(long n, long vocab) {
  if (n < 0 || vocab <= 0) return 0;
  return 4 * edf::eb_align((size_t)std::max(n, 1L) * 4) + edf::eb_align((size_t)(vocab + 1) * 4) +
         edf::eb_sort_bytes(n, vocab);
}

int edf_embedding_backward(void* stream, const int64_t* ids, const void* grad, void* grad_weight, void* workspace,
                           size_t workspace_bytes, long n, long vocab, int dim, long padding_idx, int dtype) {
  using namespace edf;
  EDF_REQUIRE(n >= 0 && n < (1L << 31) && vocab > 0 && vocab < (1L << 31) && dim > 0, EDF_ERR_INVALID_ARG,
              "need 0 <= n < 2^31 positions, 0 < vocab < 2^31 rows, dim > 0");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(grad_weight && (n == 0 || (ids && grad)), EDF_ERR_INVALID_ARG, "null tensor pointer");
  const size_t sort_bytes = eb_sort_bytes(n, vocab);
  EDF_REQUIRE(n == 0 || sort_bytes > 0, EDF_ERR_LAUNCH, "embedding backward: sort storage query failed");
  const size_t need = edf_embedding_backward_workspace_bytes(n, vocab);
  EDF_REQUIRE(workspace && workspace_bytes >= need, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes", need);
  hipStream_t s = as_stream(stream);
  return dtype == EDF_BF16 ? eb_run<bf16>(s, ids, grad, grad_weight, (char*)workspace, sort_bytes, n, vocab, dim,
                                          padding_idx)
                           : eb_run<float>(s, ids, grad, grad_weight, (char*)workspace, sort_bytes, n, vocab, dim,
                                           padding_idx);
}

}  // extern "C"
