// Streaming probe: the HBM rate a hand-written kernel reaches on this device, the ceiling
// the bandwidth-bound scans are measured against.  Not part of the product C ABI (declared
// in tests/edifice_hip_probes.h); bench.py times it beside the scans.
//
// out = in0 + in1 over n16 16-byte words (as 32-bit integer lanes; nin = 1: out = in0), every
// access 16 bytes per lane, each thread moving UNR words per loop trip with all its loads
// issued before its stores; the grid covers 256 CUs x OCC workgroups and strides over the
// buffers.
#include "edf_abi.hpp"
#include "edf_common.hpp"

namespace edf {
namespace {

typedef __attribute__((ext_vector_type(4))) unsigned u4;
constexpr int UNR = 4;

template <int NIN>
__global__ __launch_bounds__(256) void stream_probe_kernel(const u4* __restrict__ a, const u4* __restrict__ b,
                                                           u4* __restrict__ o, long n16) {
  const long stride = (long)gridDim.x * 256 * UNR;
  for (long base = (long)blockIdx.x * 256 * UNR + threadIdx.x; base < n16; base += stride) {
    u4 x[UNR], y[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const long i = base + 256L * u;
      const long j = i < n16 ? i : n16 - 1;
      x[u] = __builtin_nontemporal_load(a + j);
      if (NIN == 2) y[u] = __builtin_nontemporal_load(b + j);
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const long i = base + 256L * u;
      if (i < n16) __builtin_nontemporal_store(NIN == 2 ? x[u] + y[u] : x[u], o + i);
    }
  }
}

}  // namespace
}  // namespace edf

extern "C" int edf_probe_stream(void* stream, const void* in0, const void* in1, void* out, long n_bytes, int nin,
                                int blocks) {
  using namespace edf;
  clear_error();
  EDF_REQUIRE(in0 && out && (nin == 1 || (nin == 2 && in1)), EDF_ERR_INVALID_ARG, "null pointer or nin not 1 / 2");
  EDF_REQUIRE(n_bytes > 0 && n_bytes % 16 == 0 && blocks > 0, EDF_ERR_INVALID_ARG,
              "n_bytes must be a positive multiple of 16 and blocks positive");
  const long n16 = n_bytes / 16;
  hipStream_t s = as_stream(stream);
  if (nin == 2)
    stream_probe_kernel<2><<<blocks, 256, 0, s>>>((const u4*)in0, (const u4*)in1, (u4*)out, n16);
  else
    stream_probe_kernel<1><<<blocks, 256, 0, s>>>((const u4*)in0, nullptr, (u4*)out, n16);
  return check_launch("stream probe");
}
