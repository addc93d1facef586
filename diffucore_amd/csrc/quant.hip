// Per-row int8 activation quantization with optional ConvRot rotation (gfx950).
//
// Replaces quantize_activation / _rot_quant_kernel of the reference
// (src/diffucore/models/_int8.py:299-310, 363-406): per row,
//   scale = max(amax / 127, 1e-30),  q = clamp(rint(x / scale), -128, 127)
// with an IEEE float32 division (bit-exact with _quantize_rows, _int8.py:87-97).
//
// A row is read once, held in registers, reduced to its absmax and written as
// int8. A 256-element group goes to 8 lanes (one 16-byte load per lane per 64
// elements for 16-bit inputs). Rows of 1, 2, 4 or 8 groups fill 8 to 64 lanes
// and reduce inside the wave; other rows are packed back to back into
// workgroups and reduce segment maxima through LDS. The loads of a lane are
// all issued before any is used, and the many short wave tasks let late loads
// overlap early arithmetic. The arithmetic per element (rotation, absmax,
// code) is about 15 VALU instructions (unpack 1, butterfly 8.5, absmax 0.5,
// code 4, packing 0.75): at FLUX shapes the kernel is bound by VALU issue
// and the HBM stream together.
//
// ConvRot (group 256): x @ H_256 with H_256 = H4 (x) H4 (x) H4 (x) H4 / 16.
// The in-group index i = 64*d1 + 16*d2 + 4*d3 + d4 is split so that the
// butterfly along each base-4 digit runs without LDS:
//   d1  - the lane's 4 chunks (in registers)
//   d2  - lane bits 0,1 (quad DPP permutes)
//   d3  - lane bit 2 (ds_swizzle xor 4) and the chunk's upper/lower half
//   d4  - within 4 consecutive elements (in registers)
// Each H4 step is y[j] = S - 2*x[3-j] with S = (x0 + x1) + (x2 + x3), applied
// along d1, d2, d3, d4 in that order; the result is scaled by 1/16 (exact).
#include "common.h"

namespace dc {

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
// lane ^ 4 within each group of 32 lanes (bit-mask swizzle: and 0x1f, xor 4)
__device__ __forceinline__ float swz_xor4(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x101F));
}

// y[j] = S - 2*x[3-j], S = (x0 + x1) + (x2 + x3). 2*x is exact, so the fused
// multiply-add rounds exactly like the subtraction it replaces.
__device__ __forceinline__ float s_minus_2x(float s, float x) { return __builtin_fmaf(-2.0f, x, s); }

__device__ __forceinline__ void h4(float& x0, float& x1, float& x2, float& x3) {
  const float s = (x0 + x1) + (x2 + x3);
  const float y0 = s_minus_2x(s, x3), y1 = s_minus_2x(s, x2), y2 = s_minus_2x(s, x1), y3 = s_minus_2x(s, x0);
  x0 = y0; x1 = y1; x2 = y2; x3 = y3;
}

// H4 across the 4 lanes of each quad (lane bits 0, 1), for 8 values per lane:
// pair = x[l^1] + x[l], s = pair[l^2] + pair[l], y = s + x[l^3] * -2, the
// same operations in the same order as h4 (with the lanes of a quad in the
// roles of x0..x3), three DPP instructions per value. The compiler folds
// only some DPP moves into their users and cannot fold one into the FMA,
// whose -2 must then sit in a register: written out, the step takes 3
// instructions per value instead of 5. s_nop 1 before each group keeps two
// wait states between a VALU write and a DPP read of that register (the
// first group reads values written before the block).
__device__ __forceinline__ void h4_quad8(float (&x)[8]) {
  float p[8];
  const float m2 = -2.0f;
  asm volatile(
      "s_nop 1\n"
      "v_add_f32_dpp %0, %8, %8 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_add_f32_dpp %1, %9, %9 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_add_f32_dpp %2, %10, %10 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_add_f32_dpp %3, %11, %11 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_add_f32_dpp %4, %12, %12 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_add_f32_dpp %5, %13, %13 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_add_f32_dpp %6, %14, %14 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_add_f32_dpp %7, %15, %15 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "s_nop 1\n"
      "v_add_f32_dpp %0, %0, %0 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_add_f32_dpp %1, %1, %1 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_add_f32_dpp %2, %2, %2 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_add_f32_dpp %3, %3, %3 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_add_f32_dpp %4, %4, %4 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_add_f32_dpp %5, %5, %5 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_add_f32_dpp %6, %6, %6 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_add_f32_dpp %7, %7, %7 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_fmac_f32_dpp %0, %8, %16 quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_fmac_f32_dpp %1, %9, %16 quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_fmac_f32_dpp %2, %10, %16 quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_fmac_f32_dpp %3, %11, %16 quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_fmac_f32_dpp %4, %12, %16 quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_fmac_f32_dpp %5, %13, %16 quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_fmac_f32_dpp %6, %14, %16 quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      "v_fmac_f32_dpp %7, %15, %16 quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
      : "=&v"(p[0]), "=&v"(p[1]), "=&v"(p[2]), "=&v"(p[3]), "=&v"(p[4]), "=&v"(p[5]), "=&v"(p[6]), "=&v"(p[7])
      : "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(x[4]), "v"(x[5]), "v"(x[6]), "v"(x[7]), "v"(m2));
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = p[e];
}

// 16 * (x @ H_256) of the lane's 256-group, in place.
// v[j][e]: element 64*j + 8*q8 + e of the lane's 256-group, q8 = 2*d2 + d3hi,
// with d2 = lane & 3 and d3hi = (lane >> 2) & 1.
__device__ __forceinline__ void hadamard256(float (&v)[4][8]) {
  // d1: across the 4 chunks
#pragma unroll
  for (int e = 0; e < 8; ++e) h4(v[0][e], v[1][e], v[2][e], v[3][e]);
  // d2: lanes l, l^1, l^2, l^3
#pragma unroll
  for (int j = 0; j < 4; ++j) h4_quad8(v[j]);
  // d3 = 2*d3hi + (e >> 2): partner lane l^4 holds the other d3hi
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float xa = v[j][e], xb = v[j][e + 4];
      const float pair = xa + xb;
      const float s = pair + swz_xor4(pair);
      const float ra = swz_xor4(xa), rb = swz_xor4(xb);
      v[j][e] = s_minus_2x(s, rb);
      v[j][e + 4] = s_minus_2x(s, ra);
    }
  // d4: within 4 consecutive elements
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h4(v[j][0], v[j][1], v[j][2], v[j][3]);
    h4(v[j][4], v[j][5], v[j][6], v[j][7]);
  }
  // (the factor 1/16 is applied by the caller)
}

// ---------------------------------------------------------------- int8 codes
//
// The reference's code is clamp(rint(fl(x / s)), -128, 127) with an IEEE
// division. Every |x| <= amax and s >= fl(amax / 127), so |fl(x / s)| <= 127
// and the clamp never acts. The quotient is formed without a division by
// Markstein's correction (P. Markstein, IBM J. Res. Dev. 34(1), 1990; the
// quotient-correction theorem in Muller et al., Handbook of Floating-Point
// Arithmetic): with y = fl(1 / s) correctly rounded (one IEEE division per
// row) and q = fl(x * y), within one ulp of x / s, the residual
// r = fma(-q, s, x) is exact and fma(r, y, q) = fl(x / s), correctly rounded,
// unless something underflows. An inexact residual needs |x| < 2^-103, and
// s >= 1e-30 then puts |x / s| below 0.1: the code is 0 either way. Adding
// 1.5 * 2^23 rounds the quotient to an integer (ties to even) whose low byte
// is the two's complement code: mul, fma, fma, add per element.
//
// After the rotation the values still carry the butterfly's factor 16: the
// kernels fold the exact 1/16 into y and the 16 into s for the residual, so
// each product and residual is the unscaled one times a power of two.
constexpr float QMAGIC = 12582912.0f;              // 1.5 * 2^23

__device__ __forceinline__ uint32_t code_of(float x, float y, float s) {
  const float q = x * y;
  const float r = __builtin_fmaf(-q, s, x);
  return __float_as_uint(__builtin_fmaf(r, y, q) + QMAGIC);
}

__device__ __forceinline__ uint32_t code_exact(float x, float s) {
  return (uint32_t)(int)fminf(fmaxf(rintf(x / s), -128.0f), 127.0f);
}

// low bytes of a, b, c, d -> one word
__device__ __forceinline__ uint32_t pack4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x0c0c0400u);
  const uint32_t cd = __builtin_amdgcn_perm(d, c, 0x0c0c0400u);
  return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

// Codes of NG groups of 4 chunks (8 elements each) held by one lane, stored at
// qrow + off[n][j] for the valid chunks. The values are PRE times the ones to
// quantize (PRE = 16 after the rotation, else 1); s is the row's scale.
template <int NG, int PRE>
__device__ __forceinline__ void quantize_store(const float (&v)[NG][4][8], const bool (&ok)[NG][4],
                                               const int (&off)[NG][4], float s, int8_t* qrow) {
  const float y = (1.0f / s) * (1.0f / PRE), sp = s * (float)PRE;
#pragma unroll
  for (int n = 0; n < NG; ++n)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t w[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float* e = &v[n][j][4 * h];
        w[h] = pack4(code_of(e[0], y, sp), code_of(e[1], y, sp), code_of(e[2], y, sp), code_of(e[3], y, sp));
      }
      if (ok[n][j]) *reinterpret_cast<uint2*>(qrow + off[n][j]) = make_uint2(w[0], w[1]);
    }
}

// scale = max(amax / 127, 1e-30) from the absmax of PRE-scaled values
template <int PRE>
__device__ __forceinline__ float row_scale(float amax_pre) {
  return fmaxf((amax_pre * (1.0f / PRE)) / 127.0f, 1e-30f);
}

// ---------------------------------------------------------------- vector kernels
//
// Element layout (both kernels): a lane owns, in each 256-element group it
// covers, the 4 chunks 64*j + 8*q8 (j = 0..3) with q8 = ((r & 3) << 1) | (r >> 2),
// r = lane & 7; 8 lanes cover a group. Each chunk is one 16-byte load for
// 16-bit inputs. Needs K % 8 == 0 and 16-byte aligned rows; ROT needs K % 256 == 0.

// 8 elements from 16 (16-bit types) or 32 (float32) raw bytes
template <int DT>
__device__ __forceinline__ void unpack8(const uint4 (&r)[DT == DC_F32 ? 2 : 1], bool ok, float (&f)[8]) {
  if constexpr (DT == DC_F32) {
    const uint32_t w[8] = {r[0].x, r[0].y, r[0].z, r[0].w, r[1].x, r[1].y, r[1].z, r[1].w};
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = __uint_as_float(ok ? w[i] : 0u);
  } else {
    const uint32_t w[4] = {ok ? r[0].x : 0u, ok ? r[0].y : 0u, ok ? r[0].z : 0u, ok ? r[0].w : 0u};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = h16_to_f32<DT>(w[i] & 0xffffu);
      f[2 * i + 1] = h16_to_f32<DT>(w[i] >> 16);
    }
  }
}

// Group g0 + units * n (n < NG) of the row for the lane's unit g0 < units.
// Every load is issued, unconditionally, before any is used: chunks past the
// row (or of idle lanes) read the row's first chunk and are zeroed after.
// ZERO = false leaves the chunks of idle lanes as loaded (for kernels whose
// idle lanes' results are never read).
template <int DT, int NG, bool ZERO = true>
__device__ __forceinline__ void load_groups(const void* x, int64_t rowoff, int K, int g0, int units, int q8,
                                            float (&v)[NG][4][8], bool (&ok)[NG][4], int (&off)[NG][4]) {
  constexpr int NQ = DT == DC_F32 ? 2 : 1;
  uint4 raw[NG][4][NQ];
#pragma unroll
  for (int n = 0; n < NG; ++n)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      off[n][j] = 256 * (g0 + units * n) + 64 * j + 8 * q8;
      ok[n][j] = g0 < units && off[n][j] < K;
      const int64_t o = rowoff + (ok[n][j] ? off[n][j] : 0);
      const uint4* p = DT == DC_F32 ? reinterpret_cast<const uint4*>(static_cast<const float*>(x) + o)
                                    : reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + o);
#pragma unroll
      for (int h = 0; h < NQ; ++h) raw[n][j][h] = p[h];
    }
#pragma unroll
  for (int n = 0; n < NG; ++n)
#pragma unroll
    for (int j = 0; j < 4; ++j) unpack8<DT>(raw[n][j], ZERO ? ok[n][j] : true, v[n][j]);
}

template <int NG>
__device__ __forceinline__ float lane_amax(const float (&v)[NG][4][8]) {
  float a = 0.0f;
#pragma unroll
  for (int n = 0; n < NG; ++n)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) a = fmaxf(a, fabsf(v[n][j][e]));
  return a;
}

// max over the SEG lanes of an aligned segment (SEG = 8 .. 64)
template <int SEG>
__device__ __forceinline__ float seg_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, swz_xor4(v));
  if constexpr (SEG >= 16) v = fmaxf(v, __shfl_xor(v, 8));
  if constexpr (SEG >= 32) v = fmaxf(v, __shfl_xor(v, 16));
  if constexpr (SEG >= 64) v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}

// Rows of up to 24 groups: SEG lanes per row (256 / SEG rows per workgroup),
// NG groups per lane; the row maximum is a cross-lane reduction inside the
// wave (no LDS, no barrier).
template <int DT, int SEG, int NG, bool ROT>
__global__ void __launch_bounds__(256) quant_seg_kernel(const void* __restrict__ x, int64_t ldx, int K, int64_t M,
                                                        int8_t* __restrict__ q, int64_t ldq,
                                                        float* __restrict__ scale) {
  constexpr int RPB = 256 / SEG;
  const int t = threadIdx.x;
  const int64_t row = (int64_t)blockIdx.x * RPB + t / SEG;
  if (row >= M) return;  // a segment leaves as a whole; nothing below synchronizes
  const int li = t % SEG, r = li & 7;
  const int q8 = ((r & 3) << 1) | (r >> 2);
  float v[NG][4][8];
  bool ok[NG][4];
  int off[NG][4];
  load_groups<DT, NG>(x, row * ldx, K, li >> 3, SEG / 8, q8, v, ok, off);
  if constexpr (ROT) {
#pragma unroll
    for (int n = 0; n < NG; ++n) hadamard256(v[n]);
  }
  constexpr int PRE = ROT ? 16 : 1;
  const float s = row_scale<PRE>(seg_max<SEG>(lane_amax(v)));
  quantize_store<NG, PRE>(v, ok, off, s, q + row * ldq);
  if (li == 0) scale[row] = s;
}

// One 256-group per 8 lanes, RPB rows per workgroup (8 * G lanes each, rows
// back to back). The row maximum is reduced inside each S-lane segment
// (S = 8 * gcd(G, 8), so no segment straddles two rows), then over the row's
// G * 8 / S segment maxima in LDS. Rows past M run with their loads zeroed and
// their stores skipped, so every lane reaches the barrier.
template <int DT, int S, bool ROT>
__global__ void __launch_bounds__(1024) quant_rows_lds_kernel(const void* __restrict__ x, int64_t ldx, int K, int64_t M,
                                                              int rpb, float inv_lr, int8_t* __restrict__ q,
                                                              int64_t ldq, float* __restrict__ scale) {
  __shared__ float red[128];
  const int t = threadIdx.x, r = t & 7;
  const int G = K >> 8, lr = 8 * G;
  // t / lr: (t + 0.5) / lr is at least 0.5 / lr from an integer, far above
  // the float error for t, lr <= 1024
  const int rloc = (int)(((float)t + 0.5f) * inv_lr), li = t - rloc * lr;
  const int64_t row = (int64_t)blockIdx.x * rpb + rloc;
  const bool live = rloc < rpb && row < M;
  const int q8 = ((r & 3) << 1) | (r >> 2);
  float v[1][4][8];
  bool ok[1][4];
  int off[1][4];
  // lanes without a live row compute on row 0's values unzeroed: their
  // segment maxima fill only their own slots of red, which no live row reads
  load_groups<DT, 1, false>(x, (live ? row : 0) * ldx, K, li >> 3, live ? G : 0, q8, v, ok, off);
  if constexpr (ROT) hadamard256(v[0]);
  const float seg = seg_max<S>(lane_amax(v));
  if ((t & (S - 1)) == 0) red[t / S] = seg;
  __syncthreads();
  if (!live) return;
  const int nseg = lr / S, s0 = rloc * nseg;
  float amax = red[s0];
  for (int i = 1; i < nseg; ++i) amax = fmaxf(amax, red[s0 + i]);
  constexpr int PRE = ROT ? 16 : 1;
  const float sc = row_scale<PRE>(amax);
  quantize_store<1, PRE>(v, ok, off, sc, q + row * ldq);
  if (li == 0) scale[row] = sc;
}

// ---------------------------------------------------------------- activation + concatenation

// GELU in float32, then rounded to the 16-bit type DT as the reference rounds
// it (src/diffucore/models/_int8.py:433-435: 0.5 h (1 + erf(h / sqrt 2)),
// cast to the activation dtype; the tanh form is torch's
// gelu(approximate="tanh"), 0.5 x (1 + tanh(sqrt(2 / pi) (x + 0.044715 x^3))),
// which FLUX's MLPs use). Both are evaluated in forms without the cancellation
// the textbook forms have in the negative tail, with the hardware exp2 /
// reciprocal (this pass is VALU-bound, and the library erf / tanh cost about
// twice as much):
//   tanh form: 0.5 x (1 + tanh u) = x / (1 + 2^(-2 u log2 e));
//   erf form: 1 + erf(x / sqrt 2) = erfc(z) for x < 0, 2 - erfc(z) for x >= 0,
//   z = |x| / sqrt 2, erfc by the Chebyshev-fitted form of Press et al.,
//   Numerical Recipes (2nd ed., section 6.2, erfcc): t = 1 / (1 + z / 2),
//   erfc(z) = t exp(-z^2 - 1.26551223 + t P(t)) with P of degree 9, whose
//   relative error is below 1.2e-7 for every z >= 0.
// Both keep a small relative error over the whole line. The reference's
// cancelling forms do not: below x = -4 or so their float32 1 + erf / 1 + tanh
// sits on the 2^-24 grid, and below about -5.5 they return -0. There the
// values here are the accurate ones, so the 16-bit results can differ from the
// reference's; those elements are below 1e-4 in magnitude (codes 0 unless a
// whole row lies that far out). Elsewhere the two agree to a few float32 ulp,
// which the rounding to 16 bits hides except next to a boundary.
constexpr float LOG2E = 1.4426950408889634f;

__device__ __forceinline__ float gelu_tanh_f32(float x) {
  const float x3 = (x * x) * x;
  const float u = 0.7978845608028654f * __builtin_fmaf(0.044715f, x3, x);
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(u * (-2.0f * LOG2E)));
}

__device__ __forceinline__ float gelu_erf_f32(float x) {
  const float z = fabsf(x) * 0.7071067811865476f;
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.5f, z, 1.0f));
  float p = __builtin_fmaf(0.17087277f, t, -0.82215223f);
  p = __builtin_fmaf(p, t, 1.48851587f);
  p = __builtin_fmaf(p, t, -1.13520398f);
  p = __builtin_fmaf(p, t, 0.27886807f);
  p = __builtin_fmaf(p, t, -0.18628806f);
  p = __builtin_fmaf(p, t, 0.09678418f);
  p = __builtin_fmaf(p, t, 0.37409196f);
  p = __builtin_fmaf(p, t, 1.00002368f);
  p = __builtin_fmaf(p, t, -1.26551223f);
  const float erfc = t * __builtin_amdgcn_exp2f(__builtin_fmaf(-z, z, p) * LOG2E);
  return (0.5f * x) * (x < 0.0f ? erfc : 2.0f - erfc);
}

template <int DT>
__device__ __forceinline__ float act_round(float x, int act) {
  return round_to<DT>(act == DC_ACT_GELU_ERF ? gelu_erf_f32(x) : gelu_tanh_f32(x));
}

// Rows of concat(x1, act(x2)): columns 0 .. K1 - 1 from x1 as they are,
// columns K1 .. K - 1 from x2 through `act` (rounded to DT), then rotated and
// quantized exactly like quant_rows_lds_kernel. K1 and K are multiples of 256
// (a 256-group never straddles the two sources), so each 8-lane group unit
// reads one source.
template <int DT, int S, bool ROT, bool GEGLU>
__global__ void __launch_bounds__(1024) quant_act_rows_kernel(const void* __restrict__ x1, int64_t ld1, int K1,
                                                              const void* __restrict__ x2, int64_t ld2, int K, int act,
                                                              int64_t M, int rpb, float inv_lr,
                                                              int8_t* __restrict__ q, int64_t ldq,
                                                              float* __restrict__ scale) {
  __shared__ float red[128];
  const int t = threadIdx.x, r = t & 7;
  const int G = K >> 8, G1 = K1 >> 8, lr = 8 * G;
  const int rloc = (int)(((float)t + 0.5f) * inv_lr), li = t - rloc * lr;
  const int64_t row = (int64_t)blockIdx.x * rpb + rloc;
  const bool live = rloc < rpb && row < M;
  const int q8 = ((r & 3) << 1) | (r >> 2);
  const int g = li >> 3;
  const bool second = g >= G1;
  const int64_t rr = live ? row : 0;
  const void* src = second ? x2 : x1;
  const int64_t rowoff = second ? rr * ld2 : rr * ld1;
  float v[1][4][8];
  bool ok[1][4];
  int off[1][4];
  load_groups<DT, 1>(src, rowoff, second ? K - K1 : K1, second ? g - G1 : g, live ? (second ? G - G1 : G1) : 0, q8,
                     v, ok, off);
  if constexpr (GEGLU) {
    // x2 rows hold [value | gate], K - K1 wide each: y = round(value * round(gelu_erf(gate)))
    float gt[1][4][8];
    bool gok[1][4];
    int goff[1][4];
    load_groups<DT, 1>(src, rowoff + (second ? K - K1 : 0), second ? K - K1 : K1, second ? g - G1 : g,
                       live && second ? G - G1 : 0, q8, gt, gok, goff);
    if (second) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) v[0][j][e] = round_to<DT>(v[0][j][e] * act_round<DT>(gt[0][j][e], DC_ACT_GELU_ERF));
    }
  }
  if (second) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      off[0][j] += K1;
      if (!GEGLU && act != DC_ACT_NONE) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[0][j][e] = act_round<DT>(v[0][j][e], act);
      }
    }
  }
  if constexpr (ROT) hadamard256(v[0]);
  const float seg = seg_max<S>(lane_amax(v));
  if ((t & (S - 1)) == 0) red[t / S] = seg;
  __syncthreads();
  if (!live) return;
  const int nseg = lr / S, s0 = rloc * nseg;
  float amax = red[s0];
  for (int i = 1; i < nseg; ++i) amax = fmaxf(amax, red[s0 + i]);
  constexpr int PRE = ROT ? 16 : 1;
  const float sc = row_scale<PRE>(amax);
  quantize_store<1, PRE>(v, ok, off, sc, q + row * ldq);
  if (li == 0) scale[row] = sc;
}

// ---------------------------------------------------------------- LayerNorm-modulate + quantize

// sum over the SEG lanes of an aligned segment (xor butterfly: every lane of
// the segment ends with the same bits)
template <int SEG>
__device__ __forceinline__ float seg_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += swz_xor4(v);
  if constexpr (SEG >= 16) v += __shfl_xor(v, 8);
  if constexpr (SEG >= 32) v += __shfl_xor(v, 16);
  if constexpr (SEG >= 64) v += __shfl_xor(v, 32);
  return v;
}

// 8 16-bit values of MDT at p (16-byte aligned) as float32
template <int MDT>
__device__ __forceinline__ void load8_h16(const uint16_t* p, float (&f)[8]) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = h16_to_f32<MDT>(w[i] & 0xffffu);
    f[2 * i + 1] = h16_to_f32<MDT>(w[i] >> 16);
  }
}

// Rows of round_MDT(LayerNorm(x) * sc1 + sh), rotated and quantized like
// quant_rows_lds_kernel. LayerNorm in float32 over the row: mean = sum / K,
// then rstd = 1 / sqrt(sum((x - mean)^2) / K + eps) (two passes, no affine
// weights), y = ((x - mean) * rstd) * sc1 + sh with separate roundings, as the
// reference's _ln_mod_kernel (src/diffucore/models/_fused.py:73-85), whose
// output it rounds to the 16-bit type of sc1 / sh before the quantizer reads
// it. sc1 (the caller's 1 + scale) and sh are row row / rows_per_mod of
// [*, K] arrays, row stride ldm. Each row sum is the segment sums (xor
// butterflies) added in segment order.
template <int DT, int MDT, int S, bool ROT>
__global__ void __launch_bounds__(1024) quant_lnmod_rows_kernel(const void* __restrict__ x, int64_t ldx, int K,
                                                                int64_t M, const uint16_t* __restrict__ sc1,
                                                                const uint16_t* __restrict__ sh, int64_t ldm,
                                                                int rows_per_mod, float eps, int rpb, float inv_lr,
                                                                int8_t* __restrict__ q, int64_t ldq,
                                                                float* __restrict__ scale) {
  __shared__ float red[3][128];
  const int t = threadIdx.x, r = t & 7;
  const int G = K >> 8, lr = 8 * G;
  const int rloc = (int)(((float)t + 0.5f) * inv_lr), li = t - rloc * lr;
  const int64_t row = (int64_t)blockIdx.x * rpb + rloc;
  const bool live = rloc < rpb && row < M;
  const int q8 = ((r & 3) << 1) | (r >> 2);
  float v[1][4][8];
  bool ok[1][4];
  int off[1][4];
  load_groups<DT, 1>(x, (live ? row : 0) * ldx, K, li >> 3, live ? G : 0, q8, v, ok, off);
  // the modulation vectors for the same elements, loaded with the row
  float c[4][8], b[4][8];
  const int64_t mrow = (live ? row : 0) / rows_per_mod;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = ok[0][j] ? off[0][j] : 0;
    load8_h16<MDT>(sc1 + mrow * ldm + e, c[j]);
    load8_h16<MDT>(sh + mrow * ldm + e, b[j]);
  }
  const int nseg = lr / S, s0 = (live ? rloc : 0) * nseg;
  // mean
  float a = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) a += v[0][j][e];
  a = seg_sum<S>(a);
  if ((t & (S - 1)) == 0) red[0][t / S] = a;
  __syncthreads();
  float sum = red[0][s0];
  for (int i = 1; i < nseg; ++i) sum += red[0][s0 + i];
  const float mean = sum / (float)K;
  // centered variance (elements past the row or of idle lanes contribute 0)
  float c2 = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = ok[0][j] ? v[0][j][e] - mean : 0.0f;
      c2 += d * d;
    }
  c2 = seg_sum<S>(c2);
  if ((t & (S - 1)) == 0) red[1][t / S] = c2;
  __syncthreads();
  float var = red[1][s0];
  for (int i = 1; i < nseg; ++i) var += red[1][s0 + i];
  const float rstd = 1.0f / sqrtf(var / (float)K + eps);
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float y = round_to<MDT>(materialize(materialize((v[0][j][e] - mean) * rstd) * c[j][e]) + b[j][e]);
      v[0][j][e] = ok[0][j] ? y : 0.0f;
    }
  if constexpr (ROT) hadamard256(v[0]);
  const float seg = seg_max<S>(lane_amax(v));
  if ((t & (S - 1)) == 0) red[2][t / S] = seg;
  __syncthreads();
  if (!live) return;
  float amax = red[2][s0];
  for (int i = 1; i < nseg; ++i) amax = fmaxf(amax, red[2][s0 + i]);
  constexpr int PRE = ROT ? 16 : 1;
  const float sc = row_scale<PRE>(amax);
  quantize_store<1, PRE>(v, ok, off, sc, q + row * ldq);
  if (li == 0) scale[row] = sc;
}

// Generic path (group 0, any K, any alignment): two passes over the row.
template <int DT>
__device__ __forceinline__ float load1(const void* base, int64_t i) {
  if constexpr (DT == DC_F32) return static_cast<const float*>(base)[i];
  else return h16_to_f32<DT>(static_cast<const uint16_t*>(base)[i]);
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
  for (int64_t i = threadIdx.x; i < K; i += blockDim.x) q[row * ldq + i] = (int8_t)code_exact(load1<DT>(x, row * ldx + i), s);
  if (threadIdx.x == 0) scale[row] = s;
}

// Rows per workgroup for the row kernels (lr = 8 lanes per 256-group, S-lane
// segments): 64 / S rows make whole waves. Workgroups above 512 threads then
// give way to fewer rows when that leaves at most 1/8 of the threads idle:
// measured at FLUX's 4608 x 15360 quantize, 1 row of 480 lanes in 512
// threads runs 14% faster than 2 rows in 960 (same codes); at 3072 columns
// 1 row of 96 lanes in 128 threads (25% idle) runs 13% slower than 2 in 192.
static int rows_per_block(int lr, int S) {
  int rpb = 64 / S;
  while (rpb > 1 && rpb * lr > 1024) rpb /= 2;
  while (rpb > 1 && rpb * lr > 512) {
    const int r = rpb / 2, nt = (r * lr + 63) / 64 * 64;
    if (8 * (nt - r * lr) > nt) break;
    rpb = r;
  }
  return rpb;
}

template <int DT, int SEG, int NG, bool ROT>
static int launch_seg(const void* x, int64_t M, int K, int64_t ldx, int8_t* q, int64_t ldq, float* scale,
                      hipStream_t st) {
  constexpr int RPB = 256 / SEG;
  hipLaunchKernelGGL((quant_seg_kernel<DT, SEG, NG, ROT>), dim3((unsigned)((M + RPB - 1) / RPB)), dim3(256), 0, st,
                     x, ldx, K, M, q, ldq, scale);
  return launch_status("quant_seg_kernel");
}

template <int DT, bool ROT>
static int launch_seg_cfg(int seg, const void* x, int64_t M, int K, int64_t ldx, int8_t* q, int64_t ldq, float* scale,
                          hipStream_t st) {
  switch (seg) {
    case 8: return launch_seg<DT, 8, 1, ROT>(x, M, K, ldx, q, ldq, scale, st);
    case 16: return launch_seg<DT, 16, 1, ROT>(x, M, K, ldx, q, ldq, scale, st);
    case 32: return launch_seg<DT, 32, 1, ROT>(x, M, K, ldx, q, ldq, scale, st);
    default: return launch_seg<DT, 64, 1, ROT>(x, M, K, ldx, q, ldq, scale, st);
  }
}

template <int DT, int S, bool ROT>
static int launch_lds(const void* x, int64_t M, int K, int64_t ldx, int8_t* q, int64_t ldq, float* scale,
                      hipStream_t st) {
  const int G = K / 256, lr = 8 * G;
  const int rpb = rows_per_block(lr, S);
  const int nt = (rpb * lr + 63) / 64 * 64;
  hipLaunchKernelGGL((quant_rows_lds_kernel<DT, S, ROT>), dim3((unsigned)((M + rpb - 1) / rpb)), dim3(nt), 0, st, x,
                     ldx, K, M, rpb, 1.0f / (float)lr, q, ldq, scale);
  return launch_status("quant_rows_lds_kernel");
}

// Kernel choice: one 256-group per 8 lanes. Rows of 1, 2, 4 or 8 groups fill
// 8 to 64 lanes and reduce inside the wave; other lengths (multiples of 256,
// up to 128 groups) pack rows into workgroups and combine segment maxima in
// LDS. Many small wave tasks let the loads of late waves overlap the
// arithmetic of early ones.
template <int DT, bool ROT>
static int launch_vec(const void* x, int64_t M, int K, int64_t ldx, int8_t* q, int64_t ldq, float* scale,
                      hipStream_t st) {
  const int G = (K + 255) / 256;
  if (G == 1 || G == 2 || G == 4 || G == 8 || K % 256) {
    if (G <= 8) return launch_seg_cfg<DT, ROT>(G <= 1 ? 8 : G <= 2 ? 16 : G <= 4 ? 32 : 64, x, M, K, ldx, q, ldq,
                                               scale, st);
  }
  if (K % 256 == 0 && G <= 128) {
    switch (G % 8 == 0 ? 64 : G % 4 == 0 ? 32 : G % 2 == 0 ? 16 : 8) {
      case 64: return launch_lds<DT, 64, ROT>(x, M, K, ldx, q, ldq, scale, st);
      case 32: return launch_lds<DT, 32, ROT>(x, M, K, ldx, q, ldq, scale, st);
      case 16: return launch_lds<DT, 16, ROT>(x, M, K, ldx, q, ldq, scale, st);
      default: return launch_lds<DT, 8, ROT>(x, M, K, ldx, q, ldq, scale, st);
    }
  }
  return DC_EUNSUPPORTED;  // the caller takes the generic kernel
}

template <int DT>
static int launch_quant(const void* x, int64_t M, int64_t K, int64_t ldx, int group, int8_t* q, int64_t ldq,
                        float* scale, hipStream_t st) {
  const int eb = elem_bytes(DT);
  const bool vec = (K % 8 == 0) && aligned16(x) && ((ldx * eb) % 16 == 0) &&
                   ((reinterpret_cast<uintptr_t>(q) & 7) == 0) && (ldq % 8 == 0) && K <= 32768;
  if (group) {
    if (!vec) return fail(DC_EUNSUPPORTED, "dc_quantize_rows: the rotation needs 16-byte aligned rows and K <= 32768");
    return launch_vec<DT, true>(x, M, (int)K, ldx, q, ldq, scale, st);
  }
  if (vec) {
    const int rc = launch_vec<DT, false>(x, M, (int)K, ldx, q, ldq, scale, st);
    if (rc != DC_EUNSUPPORTED) return rc;
  }
  hipLaunchKernelGGL((quant_rows_generic<DT>), dim3((unsigned)M), dim3(256), 0, st, x, ldx, K, q, ldq, scale);
  return launch_status("quant_rows_generic");
}

template <int DT, int S, bool ROT>
static int launch_act_s(const void* x1, int64_t ld1, int K1, const void* x2, int64_t ld2, int K, int act, int64_t M,
                        int8_t* q, int64_t ldq, float* scale, hipStream_t st) {
  const int G = K / 256, lr = 8 * G;
  const int rpb = rows_per_block(lr, S);
  const int nt = (rpb * lr + 63) / 64 * 64;
  const dim3 grid((unsigned)((M + rpb - 1) / rpb));
  if (act == DC_ACT_GEGLU)
    hipLaunchKernelGGL((quant_act_rows_kernel<DT, S, ROT, true>), grid, dim3(nt), 0, st, x1, ld1, K1, x2, ld2, K, act,
                       M, rpb, 1.0f / (float)lr, q, ldq, scale);
  else
    hipLaunchKernelGGL((quant_act_rows_kernel<DT, S, ROT, false>), grid, dim3(nt), 0, st, x1, ld1, K1, x2, ld2, K,
                       act, M, rpb, 1.0f / (float)lr, q, ldq, scale);
  return launch_status("quant_act_rows_kernel");
}

template <int DT, bool ROT>
static int launch_act(const void* x1, int64_t ld1, int K1, const void* x2, int64_t ld2, int K, int act, int64_t M,
                      int8_t* q, int64_t ldq, float* scale, hipStream_t st) {
  const int G = K / 256;
  switch (G % 8 == 0 ? 64 : G % 4 == 0 ? 32 : G % 2 == 0 ? 16 : 8) {
    case 64: return launch_act_s<DT, 64, ROT>(x1, ld1, K1, x2, ld2, K, act, M, q, ldq, scale, st);
    case 32: return launch_act_s<DT, 32, ROT>(x1, ld1, K1, x2, ld2, K, act, M, q, ldq, scale, st);
    case 16: return launch_act_s<DT, 16, ROT>(x1, ld1, K1, x2, ld2, K, act, M, q, ldq, scale, st);
    default: return launch_act_s<DT, 8, ROT>(x1, ld1, K1, x2, ld2, K, act, M, q, ldq, scale, st);
  }
}

template <int DT, int MDT, bool ROT>
static int launch_lnmod(const void* x, int64_t ldx, int K, int64_t M, const void* sc1, const void* sh, int64_t ldm,
                        int rows_per_mod, float eps, int8_t* q, int64_t ldq, float* scale, hipStream_t st) {
  const int G = K / 256, lr = 8 * G;
  const int S = G % 8 == 0 ? 64 : G % 4 == 0 ? 32 : G % 2 == 0 ? 16 : 8;
  const int rpb = rows_per_block(lr, S);
  const int nt = (rpb * lr + 63) / 64 * 64;
  const dim3 grid((unsigned)((M + rpb - 1) / rpb));
  const auto* c = static_cast<const uint16_t*>(sc1);
  const auto* b = static_cast<const uint16_t*>(sh);
  const float il = 1.0f / (float)lr;
  switch (S) {
    case 64: hipLaunchKernelGGL((quant_lnmod_rows_kernel<DT, MDT, 64, ROT>), grid, dim3(nt), 0, st, x, ldx, K, M, c, b, ldm, rows_per_mod, eps, rpb, il, q, ldq, scale); break;
    case 32: hipLaunchKernelGGL((quant_lnmod_rows_kernel<DT, MDT, 32, ROT>), grid, dim3(nt), 0, st, x, ldx, K, M, c, b, ldm, rows_per_mod, eps, rpb, il, q, ldq, scale); break;
    case 16: hipLaunchKernelGGL((quant_lnmod_rows_kernel<DT, MDT, 16, ROT>), grid, dim3(nt), 0, st, x, ldx, K, M, c, b, ldm, rows_per_mod, eps, rpb, il, q, ldq, scale); break;
    default: hipLaunchKernelGGL((quant_lnmod_rows_kernel<DT, MDT, 8, ROT>), grid, dim3(nt), 0, st, x, ldx, K, M, c, b, ldm, rows_per_mod, eps, rpb, il, q, ldq, scale); break;
  }
  return launch_status("quant_lnmod_rows_kernel");
}

template <int MDT>
static int dispatch_lnmod(const void* x, int x_dtype, int64_t ldx, int K, int64_t M, const void* sc1, const void* sh,
                          int64_t ldm, int rows_per_mod, float eps, int group, int8_t* q, int64_t ldq, float* scale,
                          hipStream_t st) {
  if (x_dtype == DC_F32)
    return group ? launch_lnmod<DC_F32, MDT, true>(x, ldx, K, M, sc1, sh, ldm, rows_per_mod, eps, q, ldq, scale, st)
                 : launch_lnmod<DC_F32, MDT, false>(x, ldx, K, M, sc1, sh, ldm, rows_per_mod, eps, q, ldq, scale, st);
  return group ? launch_lnmod<MDT, MDT, true>(x, ldx, K, M, sc1, sh, ldm, rows_per_mod, eps, q, ldq, scale, st)
               : launch_lnmod<MDT, MDT, false>(x, ldx, K, M, sc1, sh, ldm, rows_per_mod, eps, q, ldq, scale, st);
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

extern "C" int dc_act_quantize_rows(const void* x1, int64_t ld1, int64_t K1, const void* x2, int64_t ld2, int64_t K2,
                                    int act, int x_dtype, int64_t M, int group, int8_t* q, int64_t ldq, float* scale,
                                    void* stream) {
  clear_error();
  const int64_t K = K1 + K2;
  const int64_t w2 = act == DC_ACT_GEGLU ? 2 * K2 : K2;   // x2 row width read
  if (M < 0 || K1 < 0 || K2 < 0 || K <= 0 || ldq < K || (K1 && ld1 < K1) || (K2 && ld2 < w2))
    return fail(DC_EINVAL, "dc_act_quantize_rows: bad M/K1/K2/ld1/ld2/ldq");
  if (M == 0) return DC_OK;
  if (M > 0x7fffffff) return fail(DC_EINVAL, "dc_act_quantize_rows: M too large");
  if ((K1 && !x1) || (K2 && !x2) || !q || !scale) return fail(DC_EINVAL, "dc_act_quantize_rows: null pointer");
  if (act != DC_ACT_NONE && act != DC_ACT_GELU_ERF && act != DC_ACT_GELU_TANH && act != DC_ACT_GEGLU)
    return fail(DC_EINVAL, "dc_act_quantize_rows: unknown act");
  if (act == DC_ACT_GEGLU && K2 == 0) return fail(DC_EINVAL, "dc_act_quantize_rows: DC_ACT_GEGLU needs K2 > 0");
  if (group != 0 && group != 256) return fail(DC_EINVAL, "dc_act_quantize_rows: group must be 0 or 256");
  if (x_dtype != DC_F16 && x_dtype != DC_BF16) return fail(DC_EINVAL, "dc_act_quantize_rows: x_dtype must be DC_F16 or DC_BF16");
  if (K1 % 256 || K2 % 256 || K > 32768)
    return fail(DC_EUNSUPPORTED, "dc_act_quantize_rows: K1 and K2 must be multiples of 256, K1 + K2 <= 32768");
  if ((K1 && (!aligned16(x1) || (ld1 * 2) % 16)) || (K2 && (!aligned16(x2) || (ld2 * 2) % 16)) ||
      (reinterpret_cast<uintptr_t>(q) & 7) || ldq % 8)
    return fail(DC_EUNSUPPORTED, "dc_act_quantize_rows: needs 16-byte aligned rows and 8-byte aligned q rows");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const void* a = K1 ? x1 : x2;
  const int64_t la = K1 ? ld1 : ld2;
  const void* b = K2 ? x2 : x1;
  const int64_t lb = K2 ? ld2 : ld1;
  if (x_dtype == DC_BF16)
    return group ? launch_act<DC_BF16, true>(a, la, (int)K1, b, lb, (int)K, act, M, q, ldq, scale, st)
                 : launch_act<DC_BF16, false>(a, la, (int)K1, b, lb, (int)K, act, M, q, ldq, scale, st);
  return group ? launch_act<DC_F16, true>(a, la, (int)K1, b, lb, (int)K, act, M, q, ldq, scale, st)
               : launch_act<DC_F16, false>(a, la, (int)K1, b, lb, (int)K, act, M, q, ldq, scale, st);
}

extern "C" int dc_ln_mod_quantize_rows(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const void* sc1,
                                       const void* shift, int mod_dtype, int64_t ldm, int64_t rows_per_mod, float eps,
                                       int group, int8_t* q, int64_t ldq, float* scale, void* stream) {
  clear_error();
  if (M < 0 || K <= 0 || ldx < K || ldq < K || ldm < K || rows_per_mod <= 0 || rows_per_mod > 0x7fffffff)
    return fail(DC_EINVAL, "dc_ln_mod_quantize_rows: bad M/K/ldx/ldq/ldm/rows_per_mod");
  if (M == 0) return DC_OK;
  if (M > 0x7fffffff) return fail(DC_EINVAL, "dc_ln_mod_quantize_rows: M too large");
  if (!x || !sc1 || !shift || !q || !scale) return fail(DC_EINVAL, "dc_ln_mod_quantize_rows: null pointer");
  if (group != 0 && group != 256) return fail(DC_EINVAL, "dc_ln_mod_quantize_rows: group must be 0 or 256");
  if (mod_dtype != DC_F16 && mod_dtype != DC_BF16)
    return fail(DC_EINVAL, "dc_ln_mod_quantize_rows: mod_dtype must be DC_F16 or DC_BF16");
  if (x_dtype != mod_dtype && x_dtype != DC_F32)
    return fail(DC_EINVAL, "dc_ln_mod_quantize_rows: x_dtype must be mod_dtype or DC_F32");
  if (!(eps >= 0.0f)) return fail(DC_EINVAL, "dc_ln_mod_quantize_rows: eps must be >= 0");
  const int eb = elem_bytes(x_dtype);
  if (K % 256 || K > 32768 || !aligned16(x) || (ldx * eb) % 16 || !aligned16(sc1) || !aligned16(shift) || ldm % 8 ||
      (reinterpret_cast<uintptr_t>(q) & 7) || ldq % 8)
    return fail(DC_EUNSUPPORTED, "dc_ln_mod_quantize_rows: needs K a multiple of 256 (<= 32768) and 16-byte aligned rows");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (mod_dtype == DC_BF16)
    return dispatch_lnmod<DC_BF16>(x, x_dtype, ldx, (int)K, M, sc1, shift, ldm, (int)rows_per_mod, eps, group, q, ldq,
                                   scale, st);
  return dispatch_lnmod<DC_F16>(x, x_dtype, ldx, (int)K, M, sc1, shift, ldm, (int)rows_per_mod, eps, group, q, ldq,
                                scale, st);
}
