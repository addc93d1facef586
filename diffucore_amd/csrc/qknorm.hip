// Per-head RMSNorm of q and k, then the rotary embedding, in one pass (gfx950).
//
// Replaces, at the producer side of the INT8 attention:
//   FLUX  QKNorm + apply_rope (flux_dit.py:129-151, 179-184):
//         n = round(round(x * rrms) * w),  rrms = rsqrt(mean(x^2) + 1e-6),
//         rotary pairs (2i, 2i+1);
//   Anima _qk_norm_rope_kernel (_fused.py:114-139):
//         n = round(w * (x * rrms)), rotary pairs (i, i + D/2);
// where round() is to the activation dtype. With a frequency table
// f [.., L, D/2, 2, 2] (float32) each pair (a, b) of normalized values becomes
//   (round(f00 a + f01 b), round(f10 a + f11 b))
// with every float32 product and sum rounded on its own (no contraction), as
// the eager torch ops and the reference's Triton kernel (fp fusion off) do.
//
// One row (a token's head, D elements) goes to D/8 lanes, 8 consecutive
// elements per lane: one 16-byte load, a sum of squares reduced across the
// row's lanes by DPP steps, 16-byte stores. A lane group takes up to 4 heads
// of one token, so the weights and the token's rotary matrices are read once
// for all of them, and each lane issues all its loads before any arithmetic.
// A workgroup of 256 threads takes 256/(D/8) lane groups. q, k and an
// optional plain copy of v (to gather two
// streams' v into one buffer for the attention) run in one launch, one
// contiguous range of workgroups each. The kernel is bound by HBM: 2 bytes
// read and 2 written per element, the weights and the frequency rows come
// from cache.
#include "common.h"

namespace dc {

struct QKSide {
  const uint16_t* x;
  uint16_t* out;
  const void* w;  // nullptr: plain copy
  int64_t sx0, sx1, sx2, so0, so1, so2;  // (B, L, H) strides in elements
};

struct QKArgs {
  QKSide s0, s1, s2;
  const float* freqs;  // nullptr: no rotary embedding
  int64_t fb, fl;      // frequency-table strides (floats) per batch, per position
  int L, H;
  int rows;            // B * L * H
  int blocks_per_side;
  int flags;           // DC_QK_* bits
  int w_f32;           // weights are float32 (else the activation dtype)
  float eps, inv_d;
};

template <int DT>
__device__ __forceinline__ void unpack8(const uint4& u, float (&v)[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = h16_to_f32<DT>(w[i] & 0xffffu);
    v[2 * i + 1] = h16_to_f32<DT>(w[i] >> 16);
  }
}

template <int DT>
__device__ __forceinline__ uint4 pack8(const float (&v)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = f32_to_h16<DT>(materialize(v[2 * i])) | (f32_to_h16<DT>(materialize(v[2 * i + 1])) << 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

template <int DT>
__device__ __forceinline__ float rnd(float x) {
  return h16_to_f32<DT>(f32_to_h16<DT>(materialize(x)));
}

// a * f0 + b * f1 with both products and the sum rounded to float32
__device__ __forceinline__ float rot(float f0, float a, float f1, float b) {
  const float p = materialize(f0 * a);
  const float q = materialize(f1 * b);
  return p + q;
}

template <int CTRL>
__device__ __forceinline__ float qk_dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
template <int PATTERN>
__device__ __forceinline__ float qk_swz(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), PATTERN));
}

// Sum over the LPR lanes of a row (aligned groups of LPR lanes), the same
// value in every lane: quad steps (lane ^ 1, lane ^ 2), then the mirrored
// lane within 8 (row_half_mirror) and within 16 (row_mirror), then lane ^ 16
// (ds_swizzle). Each step adds two equal partial sums, so all lanes agree bit
// for bit; DPP steps cost a VALU op, not an LDS round trip.
template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
  v += qk_dpp<0xB1>(v);                                // quad_perm [1,0,3,2]
  v += qk_dpp<0x4E>(v);                                // quad_perm [2,3,0,1]
  if constexpr (LPR >= 8) v += qk_dpp<0x141>(v);       // row_half_mirror
  if constexpr (LPR >= 16) v += qk_dpp<0x140>(v);      // row_mirror
  if constexpr (LPR >= 32) v += qk_swz<0x401F>(v);     // lane ^ 16 (and 0x1f, xor 0x10)
  return v;
}

// The value of lane j ^ (LPR / 2) of the same row.
template <int LPR>
__device__ __forceinline__ float partner(float v) {
  if constexpr (LPR == 4) return qk_dpp<0x4E>(v);       // lane ^ 2
  else if constexpr (LPR == 8) return qk_swz<0x101F>(v);   // lane ^ 4
  else if constexpr (LPR == 16) return qk_dpp<0x128>(v);   // row_ror:8 = lane ^ 8 within 16
  else return qk_swz<0x401F>(v);                        // lane ^ 16
}

// NH consecutive heads of one token per lane group (H % NH == 0): the
// weights and the token's rotary matrices are loaded once for all of them.
template <int DT, int LPR, int NH>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(QKArgs a) {
  constexpr int RPW = 256 / LPR;   // lane groups per workgroup
  const int side = blockIdx.x / a.blocks_per_side;
  const int blk = blockIdx.x - side * a.blocks_per_side;
  const int grp = blk * RPW + (int)threadIdx.x / LPR;   // rows NH * grp .. NH * grp + NH - 1
  const int j = (int)threadIdx.x % LPR;
  if (grp * NH >= a.rows) return;  // whole groups leave together: the lane exchanges stay inside live rows
  const QKSide s = side == 0 ? a.s0 : (side == 1 ? a.s1 : a.s2);
  const int row0 = grp * NH;
  const int h0 = row0 % a.H;
  const int bl = row0 / a.H;
  const int l = bl % a.L;
  const int b = bl / a.L;
  const uint16_t* src = s.x + b * s.sx0 + l * s.sx1 + h0 * s.sx2 + j * 8;
  uint16_t* dst = s.out + b * s.so0 + l * s.so1 + h0 * s.so2 + j * 8;
  uint4 raw[NH];
#pragma unroll
  for (int r = 0; r < NH; ++r) raw[r] = *reinterpret_cast<const uint4*>(src + r * s.sx2);
  if (s.w == nullptr) {
#pragma unroll
    for (int r = 0; r < NH; ++r) *reinterpret_cast<uint4*>(dst + r * s.so2) = raw[r];
    return;
  }
  // every load before any arithmetic: the weights, then the lane's rotary
  // matrices (pairs 4j .. 4j + 3 for adjacent pairs; for half pairs the 8
  // pairs of the lane's first-half position, shared with its partner lane)
  const bool rope = a.freqs != nullptr, half = (a.flags & DC_QK_ROPE_HALF) != 0;
  const bool lo = j < LPR / 2;
  uint4 wraw[2];
  if (a.w_f32) {
    const uint4* wp = reinterpret_cast<const uint4*>(static_cast<const float*>(s.w) + j * 8);
    wraw[0] = wp[0];
    wraw[1] = wp[1];
  } else {
    wraw[0] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(s.w) + j * 8);
    wraw[1] = wraw[0];
  }
  float4 fq[8];
  if (rope) {
    const float4* f = reinterpret_cast<const float4*>(a.freqs + b * a.fb + l * a.fl);
    if (half) {
      const int pj = lo ? j : j - LPR / 2;
#pragma unroll
      for (int i = 0; i < 8; ++i) fq[i] = f[pj * 8 + i];
    } else {
#pragma unroll
      for (int p = 0; p < 4; ++p) fq[p] = f[j * 4 + p];
    }
  }
  float w[8];
  if (a.w_f32) {
    const uint32_t wv[8] = {wraw[0].x, wraw[0].y, wraw[0].z, wraw[0].w, wraw[1].x, wraw[1].y, wraw[1].z, wraw[1].w};
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = __uint_as_float(wv[i]);
  } else {
    unpack8<DT>(wraw[0], w);
  }

#pragma unroll
  for (int r = 0; r < NH; ++r) {
    float x[8];
    unpack8<DT>(raw[r], x);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += materialize(x[i] * x[i]);
    ss = row_sum<LPR>(ss);
    const float rr = rsqrtf(ss * a.inv_d + a.eps);
    float n[8];
    if (a.flags & DC_QK_WEIGHT_F32) {
#pragma unroll
      for (int i = 0; i < 8; ++i) n[i] = rnd<DT>(w[i] * materialize(x[i] * rr));
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) n[i] = rnd<DT>(rnd<DT>(x[i] * rr) * w[i]);
    }
    if (rope) {
      float o[8];
      if (half) {
        // pair (i, i + D/2): lane j < LPR/2 holds the first halves, lane j ^ LPR/2 the second
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float m = partner<LPR>(n[i]);
          const float4 c = fq[i];
          // selects, not branches: the lower lane takes row 0 of the matrix, the upper row 1
          const float a0 = lo ? n[i] : m, b0 = lo ? m : n[i];
          o[i] = rot(lo ? c.x : c.z, a0, lo ? c.y : c.w, b0);
        }
      } else {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const float4 c = fq[p];
          o[2 * p] = rot(c.x, n[2 * p], c.y, n[2 * p + 1]);
          o[2 * p + 1] = rot(c.z, n[2 * p], c.w, n[2 * p + 1]);
        }
      }
      *reinterpret_cast<uint4*>(dst + r * s.so2) = pack8<DT>(o);
    } else {
      *reinterpret_cast<uint4*>(dst + r * s.so2) = pack8<DT>(n);
    }
  }
}

template <int DT, int LPR, int NH>
static int launch_qk(QKArgs& a, int nsides, hipStream_t st) {
  constexpr int RPW = 256 / LPR;
  const int groups = a.rows / NH;   // H % NH == 0, so rows % NH == 0
  a.blocks_per_side = (groups + RPW - 1) / RPW;
  hipLaunchKernelGGL((qk_norm_rope_kernel<DT, LPR, NH>), dim3(a.blocks_per_side * nsides), dim3(256), 0, st, a);
  return launch_status("dc_qk_norm_rope");
}

template <int DT, int LPR>
static int launch_qk_heads(QKArgs& a, int nsides, hipStream_t st) {
  if (a.H % 4 == 0) return launch_qk<DT, LPR, 4>(a, nsides, st);
  if (a.H % 2 == 0) return launch_qk<DT, LPR, 2>(a, nsides, st);
  return launch_qk<DT, LPR, 1>(a, nsides, st);
}

template <int DT>
static int dispatch_qk(QKArgs& a, int D, int nsides, hipStream_t st) {
  switch (D) {
    case 32: return launch_qk_heads<DT, 4>(a, nsides, st);
    case 64: return launch_qk_heads<DT, 8>(a, nsides, st);
    case 128: return launch_qk_heads<DT, 16>(a, nsides, st);
    default: return launch_qk_heads<DT, 32>(a, nsides, st);
  }
}

static bool strides_ok(const int64_t* s) { return s && s[0] % 8 == 0 && s[1] % 8 == 0 && s[2] % 8 == 0; }

}  // namespace dc

using namespace dc;

extern "C" int dc_qk_norm_rope(int dtype, int64_t B, int64_t L, int64_t H, int64_t D, int flags, float eps,
                               const void* q, const int64_t* q_strides, const void* q_weight,
                               const void* k, const int64_t* k_strides, const void* k_weight, int weight_dtype,
                               const float* freqs, int64_t freqs_batch_stride, int64_t freqs_pos_stride,
                               void* q_out, const int64_t* q_out_strides, void* k_out, const int64_t* k_out_strides,
                               const void* v, const int64_t* v_strides, void* v_out, const int64_t* v_out_strides,
                               void* stream) {
  clear_error();
  if (B < 0 || L < 0 || H < 0) return fail(DC_EINVAL, "dc_qk_norm_rope: negative B/L/H");
  if (dtype != DC_BF16 && dtype != DC_F16) return fail(DC_EINVAL, "dc_qk_norm_rope: dtype must be DC_F16 or DC_BF16");
  if (weight_dtype != dtype && weight_dtype != DC_F32)
    return fail(DC_EINVAL, "dc_qk_norm_rope: weight_dtype must be dtype or DC_F32");
  if (flags & ~(DC_QK_ROPE_HALF | DC_QK_WEIGHT_F32)) return fail(DC_EINVAL, "dc_qk_norm_rope: unknown flags");
  if (!(eps >= 0.0f)) return fail(DC_EINVAL, "dc_qk_norm_rope: eps must be >= 0");
  if (D != 32 && D != 64 && D != 128 && D != 256)
    return fail(DC_EUNSUPPORTED, "dc_qk_norm_rope: D must be 32, 64, 128 or 256");
  if (B * L * H > 0x7fffff00 || L > 0x7fffffff || H > 0x7fffffff)
    return fail(DC_EINVAL, "dc_qk_norm_rope: B * L * H too large");
  if (B == 0 || L == 0 || H == 0) return DC_OK;
  if (!q || !q_weight || !q_out) return fail(DC_EINVAL, "dc_qk_norm_rope: null q, q_weight or q_out");
  if ((k && (!k_weight || !k_out)) || (v && !v_out))
    return fail(DC_EINVAL, "dc_qk_norm_rope: k needs k_weight and k_out, v needs v_out");
  if (!aligned16(q) || !aligned16(q_out) || !aligned16(q_weight) || !strides_ok(q_strides) ||
      !strides_ok(q_out_strides) ||
      (k && (!aligned16(k) || !aligned16(k_out) || !aligned16(k_weight) || !strides_ok(k_strides) ||
             !strides_ok(k_out_strides))) ||
      (v && (!aligned16(v) || !aligned16(v_out) || !strides_ok(v_strides) || !strides_ok(v_out_strides))))
    return fail(DC_EUNSUPPORTED, "dc_qk_norm_rope: needs 16-byte aligned rows (strides multiples of 8 elements)");
  if (freqs && (!aligned16(freqs) || freqs_batch_stride % 4 || freqs_pos_stride % 4 || freqs_batch_stride < 0 ||
                freqs_pos_stride < 0))
    return fail(DC_EUNSUPPORTED, "dc_qk_norm_rope: freqs must be 16-byte aligned with strides multiples of 4");

  QKArgs a{};
  auto side = [](const void* x, const int64_t* sx, void* out, const int64_t* so, const void* w) {
    QKSide s;
    s.x = static_cast<const uint16_t*>(x);
    s.out = static_cast<uint16_t*>(out);
    s.w = w;
    s.sx0 = sx[0]; s.sx1 = sx[1]; s.sx2 = sx[2];
    s.so0 = so[0]; s.so1 = so[1]; s.so2 = so[2];
    return s;
  };
  QKSide sides[3];
  int n = 0;
  sides[n++] = side(q, q_strides, q_out, q_out_strides, q_weight);
  if (k) sides[n++] = side(k, k_strides, k_out, k_out_strides, k_weight);
  if (v) sides[n++] = side(v, v_strides, v_out, v_out_strides, nullptr);
  a.s0 = sides[0];
  a.s1 = n > 1 ? sides[1] : sides[0];
  a.s2 = n > 2 ? sides[2] : sides[0];
  a.freqs = freqs;
  a.fb = freqs_batch_stride;
  a.fl = freqs_pos_stride;
  a.L = (int)L;
  a.H = (int)H;
  a.rows = (int)(B * L * H);
  a.flags = flags;
  a.w_f32 = weight_dtype == DC_F32;
  a.eps = eps;
  a.inv_d = 1.0f / (float)D;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return dtype == DC_BF16 ? dispatch_qk<DC_BF16>(a, (int)D, n, st) : dispatch_qk<DC_F16>(a, (int)D, n, st);
}
