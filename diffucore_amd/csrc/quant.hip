// Per-row int8 activation quantization with optional ConvRot rotation (gfx950).
//
// Replaces quantize_activation / _rot_quant_kernel of the reference
// (src/diffucore/models/_int8.py:299-310, 363-406): per row,
//   scale = max(amax / 127, 1e-30),  q = clamp(rint(x / scale), -128, 127)
// with an IEEE float32 division (bit-exact with _quantize_rows, _int8.py:87-97).
//
// Layout: one workgroup per row. Each lane owns chunks of 8 consecutive
// elements (one 16-byte load for 16-bit inputs). HBM-bound: a row is read
// once, held in registers, reduced to its absmax and written as int8.
//
// ConvRot (group 256): x @ H_256 with H_256 = H4 (x) H4 (x) H4 (x) H4 / 16.
// The in-group index i = 64*d1 + 16*d2 + 4*d3 + d4 is split so that the
// butterfly along each base-4 digit runs without LDS:
//   d1  - the lane's 4 chunks (in registers)
//   d2  - lane bits 0,1 (quad DPP permutes)
//   d3  - lane bit 2 (ds_swizzle xor 4) and the chunk's upper/lower half
//   d4  - within 4 consecutive elements (in registers)
// Each H4 step is y[j] = S - 2*x[3-j] with S = (x0 + x1) + (x2 + x3), applied
// along d1, d2, d3, d4 in that order, then scaled by 1/16 (exact).
#include "common.h"

namespace dc {

template <int DT>
__device__ __forceinline__ void load8(const void* base, int64_t off, float (&f)[8]) {
  if constexpr (DT == DC_F32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + off);
    const float4 a = p[0], b = p[1];
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  } else {
    const uint4 u = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + off);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = h16_to_f32<DT>(w[i] & 0xffffu);
      f[2 * i + 1] = h16_to_f32<DT>(w[i] >> 16);
    }
  }
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
// lane ^ 4 within each group of 32 lanes (bit-mask swizzle: and 0x1f, xor 4)
__device__ __forceinline__ float swz_xor4(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x101F));
}

// y[j] = S - 2*x[3-j], S = (x0 + x1) + (x2 + x3)
__device__ __forceinline__ void h4(float& x0, float& x1, float& x2, float& x3) {
  const float s = (x0 + x1) + (x2 + x3);
  const float y0 = s - 2.0f * x3, y1 = s - 2.0f * x2, y2 = s - 2.0f * x1, y3 = s - 2.0f * x0;
  x0 = y0; x1 = y1; x2 = y2; x3 = y3;
}

// v[j][e]: element 64*j + 8*q8 + e of the lane's 256-group, q8 = 2*d2 + d3hi,
// with d2 = lane & 3 and d3hi = (lane >> 2) & 1.
__device__ __forceinline__ void hadamard256(float (&v)[4][8]) {
  // d1: across the 4 chunks
#pragma unroll
  for (int e = 0; e < 8; ++e) h4(v[0][e], v[1][e], v[2][e], v[3][e]);
  // d2: lanes l, l^1, l^2, l^3 (quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E, [3,2,1,0] = 0x1B)
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = v[j][e];
      const float pair = x + dpp<0xB1>(x);
      const float s = pair + dpp<0x4E>(pair);
      v[j][e] = s - 2.0f * dpp<0x1B>(x);
    }
  // d3 = 2*d3hi + (e >> 2): partner lane l^4 holds the other d3hi
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float xa = v[j][e], xb = v[j][e + 4];
      const float pair = xa + xb;
      const float s = pair + swz_xor4(pair);
      const float ra = swz_xor4(xa), rb = swz_xor4(xb);
      v[j][e] = s - 2.0f * rb;
      v[j][e + 4] = s - 2.0f * ra;
    }
  // d4: within 4 consecutive elements
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h4(v[j][0], v[j][1], v[j][2], v[j][3]);
    h4(v[j][4], v[j][5], v[j][6], v[j][7]);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) v[j][e] *= 0.0625f;
}

__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
  const int nw = blockDim.x >> 6;
  for (int i = 1; i < nw; ++i) r = fmaxf(r, red[i]);
  return r;
}

__device__ __forceinline__ uint32_t code4(float a, float b, float c, float d, float s) {
  // IEEE division then round-half-even, clamp to [-128, 127]
  const float qa = fminf(fmaxf(rintf(a / s), -128.0f), 127.0f);
  const float qb = fminf(fmaxf(rintf(b / s), -128.0f), 127.0f);
  const float qc = fminf(fmaxf(rintf(c / s), -128.0f), 127.0f);
  const float qd = fminf(fmaxf(rintf(d / s), -128.0f), 127.0f);
  return ((uint32_t)(uint8_t)(int8_t)(int)qa) | ((uint32_t)(uint8_t)(int8_t)(int)qb << 8) |
         ((uint32_t)(uint8_t)(int8_t)(int)qc << 16) | ((uint32_t)(uint8_t)(int8_t)(int)qd << 24);
}

// Vector path: K % 8 == 0, 16-byte aligned rows. NJ chunks of 8 per lane.
template <int DT, int NJ, bool ROT>
__global__ void __launch_bounds__(1024) quant_rows_kernel(const void* __restrict__ x, int64_t ldx, int K,
                                                          int8_t* __restrict__ q, int64_t ldq,
                                                          float* __restrict__ scale) {
  __shared__ float red[16];
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x, nt = blockDim.x;
  int off[NJ];
  bool ok[NJ];
  if constexpr (ROT) {
    static_assert(NJ == 4, "the rotation layout owns 4 chunks per lane");
    const int g = t >> 3, r = t & 7;
    const int q8 = ((r & 3) << 1) | (r >> 2);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      off[j] = 256 * g + 64 * j + 8 * q8;
      ok[j] = 256 * g < K;
    }
  } else {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      off[j] = 8 * (t + j * nt);
      ok[j] = off[j] < K;
    }
  }
  float v[NJ][8];
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    if (ok[j]) {
      load8<DT>(x, row * ldx + off[j], v[j]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[j][e] = 0.0f;
    }
  }
  if constexpr (ROT) hadamard256(v);
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[j][e]));
  amax = block_max(amax, red);
  const float s = fmaxf(amax / 127.0f, 1e-30f);
  int8_t* qrow = q + row * ldq;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    if (!ok[j]) continue;
    uint2 out;
    out.x = code4(v[j][0], v[j][1], v[j][2], v[j][3], s);
    out.y = code4(v[j][4], v[j][5], v[j][6], v[j][7], s);
    *reinterpret_cast<uint2*>(qrow + off[j]) = out;
  }
  if (t == 0) scale[row] = s;
}

// Generic path (group 0, any K, any alignment): two passes over the row.
template <int DT>
__device__ __forceinline__ float load1(const void* base, int64_t i) {
  if constexpr (DT == DC_F32) return static_cast<const float*>(base)[i];
  else return h16_to_f32<DT>(static_cast<const uint16_t*>(base)[i]);
}

template <int DT>
__global__ void __launch_bounds__(256) quant_rows_generic(const void* __restrict__ x, int64_t ldx, int64_t K,
                                                          int8_t* __restrict__ q, int64_t ldq,
                                                          float* __restrict__ scale) {
  __shared__ float red[16];
  const int64_t row = blockIdx.x;
  float amax = 0.0f;
  for (int64_t i = threadIdx.x; i < K; i += blockDim.x) amax = fmaxf(amax, fabsf(load1<DT>(x, row * ldx + i)));
  amax = block_max(amax, red);
  const float s = fmaxf(amax / 127.0f, 1e-30f);
  for (int64_t i = threadIdx.x; i < K; i += blockDim.x) {
    const float v = fminf(fmaxf(rintf(load1<DT>(x, row * ldx + i) / s), -128.0f), 127.0f);
    q[row * ldq + i] = (int8_t)(int)v;
  }
  if (threadIdx.x == 0) scale[row] = s;
}

template <int DT>
static int launch_quant(const void* x, int64_t M, int64_t K, int64_t ldx, int group, int8_t* q, int64_t ldq,
                        float* scale, hipStream_t st) {
  const int eb = elem_bytes(DT);
  const bool vec = (K % 8 == 0) && aligned16(x) && ((ldx * eb) % 16 == 0) &&
                   ((reinterpret_cast<uintptr_t>(q) & 7) == 0) && (ldq % 8 == 0) && K <= 32768;
  if (group) {
    if (!vec) return fail(DC_EUNSUPPORTED, "dc_quantize_rows: the rotation needs 16-byte aligned rows and K <= 32768");
    const int nt = (int)(((K / 32) + 63) / 64 * 64);
    hipLaunchKernelGGL((quant_rows_kernel<DT, 4, true>), dim3((unsigned)M), dim3(nt), 0, st, x, ldx, (int)K, q, ldq,
                       scale);
    return launch_status("quant_rows_kernel<rot>");
  }
  if (!vec) {
    hipLaunchKernelGGL((quant_rows_generic<DT>), dim3((unsigned)M), dim3(256), 0, st, x, ldx, K, q, ldq, scale);
    return launch_status("quant_rows_generic");
  }
  const int64_t nch = K / 8;
  if (nch <= 256) {
    const int nt = (int)((nch + 63) / 64 * 64);
    hipLaunchKernelGGL((quant_rows_kernel<DT, 1, false>), dim3((unsigned)M), dim3(nt), 0, st, x, ldx, (int)K, q,
                       ldq, scale);
  } else if (nch <= 2048) {
    const int nt = (int)(((nch + 1) / 2 + 63) / 64 * 64);
    hipLaunchKernelGGL((quant_rows_kernel<DT, 2, false>), dim3((unsigned)M), dim3(nt), 0, st, x, ldx, (int)K, q,
                       ldq, scale);
  } else {
    const int nt = (int)(((nch + 3) / 4 + 63) / 64 * 64);
    hipLaunchKernelGGL((quant_rows_kernel<DT, 4, false>), dim3((unsigned)M), dim3(nt), 0, st, x, ldx, (int)K, q,
                       ldq, scale);
  }
  return launch_status("quant_rows_kernel");
}

}  // namespace dc

using namespace dc;

extern "C" int dc_quantize_rows(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, int group, int8_t* q,
                                int64_t ldq, float* scale, void* stream) {
  clear_error();
  if (M < 0 || K <= 0 || ldx < K || ldq < K) return fail(DC_EINVAL, "dc_quantize_rows: bad M/K/ldx/ldq");
  if (M == 0) return DC_OK;
  if (M > 0x7fffffff) return fail(DC_EINVAL, "dc_quantize_rows: M too large");
  if (!x || !q || !scale) return fail(DC_EINVAL, "dc_quantize_rows: null pointer");
  if (group != 0 && group != 256) return fail(DC_EINVAL, "dc_quantize_rows: group must be 0 or 256");
  if (group && K % group) return fail(DC_EINVAL, "dc_quantize_rows: K is not a multiple of the ConvRot group");
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (x_dtype) {
    case DC_F16: return launch_quant<DC_F16>(x, M, K, ldx, group, q, ldq, scale, st);
    case DC_BF16: return launch_quant<DC_BF16>(x, M, K, ldx, group, q, ldq, scale, st);
    case DC_F32: return launch_quant<DC_F32>(x, M, K, ldx, group, q, ldq, scale, st);
    default: return fail(DC_EINVAL, "dc_quantize_rows: x_dtype must be DC_F16, DC_BF16 or DC_F32");
  }
}
