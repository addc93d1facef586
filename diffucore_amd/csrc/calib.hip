// MFMA throughput calibration (no counterpart in the reference): the rate this
// device's matrix cores sustain on back-to-back independent MFMAs of the two
// shapes the hot path runs, v_mfma_i32_32x32x32_i8 (QK^T and the W8A8 GEMM)
// and v_mfma_f32_32x32x16_bf16 (PV), with nothing else in the loop. The
// caller times a launch and divides the work by the time (bench.py
// --mfma-ceiling); the published peak assumes every matrix core busy every
// cycle at the peak engine clock, which the chip does not hold under this
// load, and with operands that change from one MFMA to the next (as real data
// does) it draws more power and clocks lower than with constant operands.
//
// Each wave keeps 4 accumulators (independent chains, so MFMAs issue back to
// back) and 8 operand pairs; `vary` = 0 reuses one pair, 1 cycles through the
// 8, whose values are a per-lane hash (int8: uniform codes; bf16: values in
// magnitudes in [0.5, 2)). One workgroup per compute unit (its dynamic LDS keeps a second off
// the unit), `waves` waves per SIMD.
#include "common.h"

#include <mutex>

namespace dc {

__device__ __forceinline__ uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352dU;
  x ^= x >> 15;
  x *= 0x846ca68bU;
  x ^= x >> 16;
  return x;
}

template <int KIND, bool VARY>
__global__ void __launch_bounds__(512) mfma_probe_kernel(int iters, int* __restrict__ sink) {
  const uint32_t lane = threadIdx.x & 63;
  v4i a[8], b[8];
#pragma unroll
  for (int s = 0; s < 8; ++s)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      uint32_t ha = mix32(lane * 977u + s * 131u + e * 7u + 1u), hb = mix32(lane * 613u + s * 89u + e * 13u + 2u);
      if (KIND == 1) {
        // two bf16 values per register, magnitudes in [0.5, 2): random sign,
        // exponent 126 or 127, random mantissa
        ha = (ha & 0x80ff80ffu) | 0x3f003f00u;
        hb = (hb & 0x80ff80ffu) | 0x3f003f00u;
      }
      a[s][e] = (int)ha;
      b[s][e] = (int)hb;
    }
  v16i ia[4];
  v16f fa[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    ia[c] = v16i{0};
    fa[c] = v16f{0.f};
  }
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int sa = VARY ? k : 0, sb = VARY ? (3 * k + 1) & 7 : 0;
      if constexpr (KIND == 0)
        ia[k & 3] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[sa], b[sb], ia[k & 3], 0, 0, 0);
      else
        fa[k & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a[sa]),
                                                            __builtin_bit_cast(v8bf, b[sb]), fa[k & 3], 0, 0, 0);
    }
  }
  int s = 0;
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int j = 0; j < 16; ++j) s += KIND == 0 ? ia[c][j] : (int)fa[c][j];
  if (lane == 0) sink[blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6)] = s;
}

template <int KIND, bool VARY>
static int launch_probe(int blocks, int threads, int iters, int* sink, hipStream_t st) {
  constexpr size_t LDS = 96 * 1024;   // more than half the unit's LDS: one workgroup per CU
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [] {
    attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&mfma_probe_kernel<KIND, VARY>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS);
  });
  if (attr != hipSuccess) {
    set_error("dc_mfma_probe: %s", hipGetErrorString(attr));
    return DC_EHIP;
  }
  hipLaunchKernelGGL((mfma_probe_kernel<KIND, VARY>), dim3((unsigned)blocks), dim3((unsigned)threads), LDS, st, iters,
                     sink);
  return launch_status("mfma_probe_kernel");
}

}  // namespace dc

using namespace dc;

extern "C" int dc_mfma_probe(int kind, int vary, int waves, int iters, int* sink, void* stream) {
  clear_error();
  if ((kind != 0 && kind != 1) || (vary != 0 && vary != 1) || (waves != 1 && waves != 2) || iters <= 0)
    return fail(DC_EINVAL, "dc_mfma_probe: kind 0 or 1, vary 0 or 1, waves 1 or 2, iters > 0");
  if (!sink) return fail(DC_EINVAL, "dc_mfma_probe: null pointer");
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                              hipSuccess || cus <= 0)
    return fail(DC_EHIP, "dc_mfma_probe: no device");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int threads = 256 * waves;
  if (kind == 0)
    return vary ? launch_probe<0, true>(cus, threads, iters, sink, st) : launch_probe<0, false>(cus, threads, iters, sink, st);
  return vary ? launch_probe<1, true>(cus, threads, iters, sink, st) : launch_probe<1, false>(cus, threads, iters, sink, st);
}

extern "C" int dc_mfma_probe_units(void) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                              hipSuccess)
    return 0;
  return cus;
}
