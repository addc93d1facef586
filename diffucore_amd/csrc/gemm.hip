// W8A8 GEMM on int8 MFMA with a fused rescale / bias / cast epilogue (gfx950).
//
// Replaces the reference's int_mm + rescale (src/diffucore/models/_int8.py:200-207,
// 313-323) and its Turing-only fused scaled_mm (kernels/int8_gemm_sm75.cu:25-88).
// The epilogue rounds exactly like rescale(int_mm(q, w), sx, sw, bias, dtype):
//   y = cast(float(acc) * (sx[m] * sw[n]));  y = cast(float(y) + float(cast(bias[n])))
//
// Work split: C^T = W . A^T on v_mfma_i32_32x32x32_i8, so each lane's
// accumulators belong to one activation row m and 4 consecutive output
// channels n per register quad (8- or 16-byte stores in the epilogue).
//   workgroup tile  BN x BM = (64*FN) x (64*FM), 4 waves as 2 (n) x 2 (m)
//   wave tile       (32*FN) x (32*FM) = FN x FM MFMA blocks of 32 x 32
//   k step          64 bytes per LDS stage, two stages, register-staged loads
// LDS rows are 64 bytes (four 16-byte chunks); chunk c of row r sits at
// c ^ ((r >> 1) & 3) so the 32 rows an MFMA operand read touches spread over
// all banks. Tiles are ordered so each XCD (8 per device; the hardware deals
// workgroups round-robin over them) works a contiguous, L2-friendly range.
#include "common.h"

namespace dc {

struct GemmArgs {
  const int8_t* a;
  const int8_t* w;
  const float* sx;
  const float* sw;
  const void* bias;
  void* out;
  int64_t lda, ldw, ldo;
  int M, N, K;
  int tiles_m, tiles_n;
  int vec_out;  // 1 when 4-wide output stores are aligned
};

constexpr int BK = 64;
constexpr int GROUP_M = 8;

__device__ __forceinline__ int swz64(int c, int r) { return c ^ ((r >> 1) & 3); }

template <int BIAS_DT>
__device__ __forceinline__ float load_bias(const void* b, int n) {
  if constexpr (BIAS_DT == DC_F32) return static_cast<const float*>(b)[n];
  else return h16_to_f32<BIAS_DT>(static_cast<const uint16_t*>(b)[n]);
}

template <int OUT_DT, int BIAS_DT>
__device__ __forceinline__ float epi(int acc, float sxm, float swn, const void* bias, int n) {
  float y = round_to<OUT_DT>(materialize((float)acc * (sxm * swn)));
  if constexpr (BIAS_DT != DC_NONE)
    y = round_to<OUT_DT>(materialize(y + round_to<OUT_DT>(load_bias<BIAS_DT>(bias, n))));
  return y;
}

template <int OUT_DT>
__device__ __forceinline__ void store1(void* out, int64_t idx, float y) {
  if constexpr (OUT_DT == DC_F32) static_cast<float*>(out)[idx] = y;
  else static_cast<uint16_t*>(out)[idx] = (uint16_t)f32_to_h16<OUT_DT>(y);
}

template <int FN, int FM, int OUT_DT, int BIAS_DT>
__global__ void __launch_bounds__(256, 1) w8a8_gemm_kernel(GemmArgs p) {
  constexpr int BN = 64 * FN, BM = 64 * FM;
  constexpr int WCH = BN * BK / 16, ACH = BM * BK / 16;  // 16-byte chunks per stage
  constexpr int NWL = WCH / 256, NAL = ACH / 256;
  static_assert(WCH % 256 == 0 && ACH % 256 == 0, "tile must split evenly over 256 threads");
  __shared__ __attribute__((aligned(16))) int8_t sw_lds[2][BN * BK];
  __shared__ __attribute__((aligned(16))) int8_t sa_lds[2][BM * BK];

  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int l32 = lane & 31, hf = lane >> 5;

  // tile order: XCD-contiguous ranges, then GROUP_M m-tiles per n sweep
  const int nwg = gridDim.x, wg = blockIdx.x;
  const int logical = (nwg % 8 == 0) ? (wg % 8) * (nwg / 8) + wg / 8 : wg;
  const int per_group = GROUP_M * p.tiles_n;
  const int grp = logical / per_group;
  const int first_m = grp * GROUP_M;
  const int gsize = min(p.tiles_m - first_m, GROUP_M);
  const int tm = first_m + (logical % per_group) % gsize;
  const int tn = (logical % per_group) / gsize;
  const int m0 = tm * BM, n0 = tn * BN;

  const int wn = wv & 1, wm = wv >> 1;
  const int nb = wn * 32 * FN, mb = wm * 32 * FM;

  v16i acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = v16i{0};

  uint4 wreg[NWL], areg[NAL];
  const int nk = (p.K + BK - 1) / BK;

  auto gload = [&](int kt) {
    const int k0 = kt * BK;
#pragma unroll
    for (int u = 0; u < NWL; ++u) {
      const int ci = t + u * 256, r = ci >> 2, c = ci & 3;
      const int n = n0 + r, k = k0 + 16 * c;
      wreg[u] = (n < p.N && k < p.K) ? *reinterpret_cast<const uint4*>(p.w + (int64_t)n * p.ldw + k)
                                     : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < NAL; ++u) {
      const int ci = t + u * 256, r = ci >> 2, c = ci & 3;
      const int m = m0 + r, k = k0 + 16 * c;
      areg[u] = (m < p.M && k < p.K) ? *reinterpret_cast<const uint4*>(p.a + (int64_t)m * p.lda + k)
                                     : make_uint4(0, 0, 0, 0);
    }
  };
  auto sstore = [&](int stage) {
#pragma unroll
    for (int u = 0; u < NWL; ++u) {
      const int ci = t + u * 256, r = ci >> 2, c = ci & 3;
      *reinterpret_cast<uint4*>(&sw_lds[stage][r * BK + swz64(c, r) * 16]) = wreg[u];
    }
#pragma unroll
    for (int u = 0; u < NAL; ++u) {
      const int ci = t + u * 256, r = ci >> 2, c = ci & 3;
      *reinterpret_cast<uint4*>(&sa_lds[stage][r * BK + swz64(c, r) * 16]) = areg[u];
    }
  };

  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int st = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      const int c = 2 * ks + hf;
      v4i wf[FN], af[FM];
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        const int r = nb + 32 * i + l32;
        wf[i] = *reinterpret_cast<const v4i*>(&sw_lds[st][r * BK + swz64(c, r) * 16]);
      }
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const int r = mb + 32 * j + l32;
        af[j] = *reinterpret_cast<const v4i*>(&sa_lds[st][r * BK + swz64(c, r) * 16]);
      }
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[i], af[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) sstore(st ^ 1);
    __syncthreads();
  }

  // epilogue: acc[i][j] register r -> n = n0 + nb + 32 i + 8 (r / 4) + 4 hf + r % 4, m = m0 + mb + 32 j + l32
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int m = m0 + mb + 32 * j + l32;
    if (m >= p.M) continue;
    float sxm = 0.0f;
    if constexpr (OUT_DT != DC_I32) sxm = p.sx[m];
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + nb + 32 * i + 8 * g + 4 * hf;
        if (n >= p.N) continue;
        const int64_t base = (int64_t)m * p.ldo + n;
        const int a0 = acc[i][j][4 * g], a1 = acc[i][j][4 * g + 1], a2 = acc[i][j][4 * g + 2], a3 = acc[i][j][4 * g + 3];
        if constexpr (OUT_DT == DC_I32) {
          int* o = static_cast<int*>(p.out);
          if (p.vec_out && n + 3 < p.N) {
            *reinterpret_cast<int4*>(o + base) = make_int4(a0, a1, a2, a3);
          } else {
            const int av[4] = {a0, a1, a2, a3};
            for (int e = 0; e < 4 && n + e < p.N; ++e) o[base + e] = av[e];
          }
        } else {
          if (p.vec_out && n + 3 < p.N) {
            const float4 s4 = *reinterpret_cast<const float4*>(p.sw + n);
            const float y0 = epi<OUT_DT, BIAS_DT>(a0, sxm, s4.x, p.bias, n);
            const float y1 = epi<OUT_DT, BIAS_DT>(a1, sxm, s4.y, p.bias, n + 1);
            const float y2 = epi<OUT_DT, BIAS_DT>(a2, sxm, s4.z, p.bias, n + 2);
            const float y3 = epi<OUT_DT, BIAS_DT>(a3, sxm, s4.w, p.bias, n + 3);
            if constexpr (OUT_DT == DC_F32) {
              *reinterpret_cast<float4*>(static_cast<float*>(p.out) + base) = make_float4(y0, y1, y2, y3);
            } else {
              const uint32_t lo = f32_to_h16<OUT_DT>(y0) | (f32_to_h16<OUT_DT>(y1) << 16);
              const uint32_t hi = f32_to_h16<OUT_DT>(y2) | (f32_to_h16<OUT_DT>(y3) << 16);
              *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.out) + base) = make_uint2(lo, hi);
            }
          } else {
            const int av[4] = {a0, a1, a2, a3};
            for (int e = 0; e < 4 && n + e < p.N; ++e)
              store1<OUT_DT>(p.out, base + e, epi<OUT_DT, BIAS_DT>(av[e], sxm, p.sw[n + e], p.bias, n + e));
          }
        }
      }
  }
}

// Rescale pass over an int32 accumulator (dc_rescale): one thread per 4 outputs.
template <int OUT_DT, int BIAS_DT>
__global__ void __launch_bounds__(256) rescale_kernel(const int32_t* __restrict__ acc, int64_t lda,
                                                      const float* __restrict__ sx, const float* __restrict__ sw,
                                                      const void* __restrict__ bias, void* __restrict__ out,
                                                      int64_t ldo, int M, int N) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int n4 = (N + 3) / 4;
  const int64_t m = idx / n4;
  const int n = (int)(idx % n4) * 4;
  if (m >= M) return;
  const float sxm = sx[m];
  for (int e = 0; e < 4 && n + e < N; ++e)
    store1<OUT_DT>(out, m * ldo + n + e, epi<OUT_DT, BIAS_DT>(acc[m * lda + n + e], sxm, sw[n + e], bias, n + e));
}

template <int FN, int FM, int OUT_DT, int BIAS_DT>
static int launch_gemm(GemmArgs p, hipStream_t st) {
  p.tiles_n = (p.N + 64 * FN - 1) / (64 * FN);
  p.tiles_m = (p.M + 64 * FM - 1) / (64 * FM);
  const int64_t tiles = (int64_t)p.tiles_n * p.tiles_m;
  if (tiles > 0x7fffffff) return fail(DC_EINVAL, "dc_w8a8_gemm: problem too large");
  hipLaunchKernelGGL((w8a8_gemm_kernel<FN, FM, OUT_DT, BIAS_DT>), dim3((unsigned)tiles), dim3(256), 0, st, p);
  return launch_status("w8a8_gemm_kernel");
}

template <int OUT_DT, int BIAS_DT>
static int pick_tile(GemmArgs p, hipStream_t st) {
  // 256 x 256 tiles while they fill the device; smaller tiles for small problems
  const int64_t big = (int64_t)((p.N + 255) / 256) * ((p.M + 255) / 256);
  if (big >= 192) return launch_gemm<4, 4, OUT_DT, BIAS_DT>(p, st);
  return launch_gemm<2, 2, OUT_DT, BIAS_DT>(p, st);
}

template <int OUT_DT>
static int dispatch_bias(GemmArgs p, int bias_dtype, hipStream_t st) {
  switch (bias_dtype) {
    case DC_NONE: return pick_tile<OUT_DT, DC_NONE>(p, st);
    case DC_F16: return pick_tile<OUT_DT, DC_F16>(p, st);
    case DC_BF16: return pick_tile<OUT_DT, DC_BF16>(p, st);
    case DC_F32: return pick_tile<OUT_DT, DC_F32>(p, st);
    default: return fail(DC_EINVAL, "dc_w8a8_gemm: bad bias_dtype");
  }
}

template <int OUT_DT, int BIAS_DT>
static int launch_rescale(const int32_t* acc, int64_t lda, const float* sx, const float* sw, const void* bias,
                          void* out, int64_t ldo, int64_t M, int64_t N, hipStream_t st) {
  const int64_t n = M * ((N + 3) / 4);
  hipLaunchKernelGGL((rescale_kernel<OUT_DT, BIAS_DT>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, acc, lda,
                     sx, sw, bias, out, ldo, (int)M, (int)N);
  return launch_status("rescale_kernel");
}

template <int OUT_DT>
static int rescale_bias(const int32_t* acc, int64_t lda, const float* sx, const float* sw, const void* bias,
                        int bias_dtype, void* out, int64_t ldo, int64_t M, int64_t N, hipStream_t st) {
  switch (bias_dtype) {
    case DC_NONE: return launch_rescale<OUT_DT, DC_NONE>(acc, lda, sx, sw, bias, out, ldo, M, N, st);
    case DC_F16: return launch_rescale<OUT_DT, DC_F16>(acc, lda, sx, sw, bias, out, ldo, M, N, st);
    case DC_BF16: return launch_rescale<OUT_DT, DC_BF16>(acc, lda, sx, sw, bias, out, ldo, M, N, st);
    case DC_F32: return launch_rescale<OUT_DT, DC_F32>(acc, lda, sx, sw, bias, out, ldo, M, N, st);
    default: return fail(DC_EINVAL, "dc_rescale: bad bias_dtype");
  }
}

}  // namespace dc

using namespace dc;

extern "C" int dc_w8a8_gemm(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, const float* sx,
                            const float* sw, const void* bias, int bias_dtype, void* out, int out_dtype, int64_t ldo,
                            int64_t M, int64_t N, int64_t K, void* stream) {
  clear_error();
  if (M < 0 || N < 0 || K < 0) return fail(DC_EINVAL, "dc_w8a8_gemm: negative size");
  if (M == 0 || N == 0) return DC_OK;
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff) return fail(DC_EINVAL, "dc_w8a8_gemm: size too large");
  if (!a || !w || !out) return fail(DC_EINVAL, "dc_w8a8_gemm: null pointer");
  if (K == 0) return fail(DC_EINVAL, "dc_w8a8_gemm: K must be positive");
  if (K % 16 || lda % 16 || ldw % 16 || lda < K || ldw < K || !aligned16(a) || !aligned16(w))
    return fail(DC_EUNSUPPORTED, "dc_w8a8_gemm: needs K, lda, ldw multiples of 16 and 16-byte aligned a, w");
  if (ldo < N) return fail(DC_EINVAL, "dc_w8a8_gemm: ldo < N");
  if (out_dtype != DC_I32 && (!sx || !sw)) return fail(DC_EINVAL, "dc_w8a8_gemm: scales are required");
  if (bias_dtype != DC_NONE && !bias) return fail(DC_EINVAL, "dc_w8a8_gemm: bias_dtype given without bias");
  GemmArgs p{};
  p.a = a; p.w = w; p.sx = sx; p.sw = sw; p.bias = bias; p.out = out;
  p.lda = lda; p.ldw = ldw; p.ldo = ldo;
  p.M = (int)M; p.N = (int)N; p.K = (int)K;
  const int ob = elem_bytes(out_dtype);
  p.vec_out = ((reinterpret_cast<uintptr_t>(out) % (4 * (uintptr_t)(ob ? ob : 1))) == 0) && (ldo % 4 == 0) &&
              (out_dtype == DC_I32 || (reinterpret_cast<uintptr_t>(sw) & 15) == 0);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (out_dtype) {
    case DC_I32: return pick_tile<DC_I32, DC_NONE>(p, st);
    case DC_F16: return dispatch_bias<DC_F16>(p, bias_dtype, st);
    case DC_BF16: return dispatch_bias<DC_BF16>(p, bias_dtype, st);
    case DC_F32: return dispatch_bias<DC_F32>(p, bias_dtype, st);
    default: return fail(DC_EINVAL, "dc_w8a8_gemm: bad out_dtype");
  }
}

extern "C" int dc_rescale(const int32_t* acc, int64_t lda, const float* sx, const float* sw, const void* bias,
                          int bias_dtype, void* out, int out_dtype, int64_t ldo, int64_t M, int64_t N, void* stream) {
  clear_error();
  if (M < 0 || N < 0) return fail(DC_EINVAL, "dc_rescale: negative size");
  if (M == 0 || N == 0) return DC_OK;
  if (!acc || !sx || !sw || !out) return fail(DC_EINVAL, "dc_rescale: null pointer");
  if (lda < N || ldo < N) return fail(DC_EINVAL, "dc_rescale: leading dimension < N");
  if (bias_dtype != DC_NONE && !bias) return fail(DC_EINVAL, "dc_rescale: bias_dtype given without bias");
  if (M * ((N + 3) / 4) > (int64_t)0x7fffffff * 256) return fail(DC_EINVAL, "dc_rescale: too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (out_dtype) {
    case DC_F16: return rescale_bias<DC_F16>(acc, lda, sx, sw, bias, bias_dtype, out, ldo, M, N, st);
    case DC_BF16: return rescale_bias<DC_BF16>(acc, lda, sx, sw, bias, bias_dtype, out, ldo, M, N, st);
    case DC_F32: return rescale_bias<DC_F32>(acc, lda, sx, sw, bias, bias_dtype, out, ldo, M, N, st);
    default: return fail(DC_EINVAL, "dc_rescale: bad out_dtype");
  }
}
