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
//   workgroup tile  BN x BM = (32*WN*FN) x (32*WM*FM), WN x WM waves
//   wave tile       (32*FN) x (32*FM) = FN x FM MFMA blocks of 32 x 32
//   k depth         128 bytes per LDS stage, two stages
// Four instantiations: 256 x 256 tiles on 8 waves (2 along n x 4 along m,
// each 128 x 64), 192 x 256 on 8 waves (each 96 x 64), 192 x 128 on 4 waves
// (each 96 x 64) and 128 x 128 on 4 waves (each 64 x 64); pick_tile chooses
// by how full the last round of tiles is.
// 256 x 256 tiles with K % 256 == 0 go to w8a8_gemm_dma_kernel instead (4
// waves of 128 x 128, operands loaded straight into LDS; described there).
// Pipeline per 128-byte k tile (4 MFMA k-steps): operand fragments for the
// next k-step are read from LDS while the current one's MFMAs run; the next
// tile, staged in registers, is written to the other LDS stage after the first
// k-step; the tile after that is fetched from global memory after the second.
// LDS rows are padded from 128 to 144 bytes so the 32 rows an operand read
// touches spread over all banks, and every read address is a per-lane base
// plus an immediate. Tiles are ordered so each XCD (8 per device; the hardware
// deals workgroups round-robin over them) works a contiguous, L2-friendly range.
#include "common.h"

#include <atomic>

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
  int vec16;    // 1 when 16-byte output stores at multiples of 16 bytes into a row are aligned
  // split-K (int32 partials only): blockIdx.y takes k in [y * kslice, (y + 1) * kslice)
  // and writes its partial sums at out + y * split_stride
  int ksplit, kslice;
  int64_t split_stride;
  // gated residual (dc_w8a8_gemm_grouped_gated; DMA-fed kernel only):
  // out = res + gate * y, res [M, N] with row stride ldr, gate [N], both of
  // the output dtype
  const void* res;
  const void* gate;
  int64_t ldr;
};

// One problem of a grouped launch (dc_w8a8_gemm_grouped): the per-problem
// fields of GemmArgs.
struct GroupProblem {
  const int8_t* a;
  const int8_t* w;
  const float* sx;
  const float* sw;
  const void* bias;
  void* out;
  int64_t lda, ldw, ldo;
  int M, tiles_m, vec_out, vec16;
  const void* res;
  const void* gate;
  int64_t ldr;
};

// A grouped launch of the DMA-fed kernel: problem g owns logical tiles
// first[g] .. first[g + 1] - 1. ngroup == 0: one problem, all in GemmArgs.
struct GroupArgs {
  int ngroup;
  int first[DC_GEMM_MAX_GROUP + 1];
  GroupProblem prob[DC_GEMM_MAX_GROUP];
};

constexpr int BK = 128;            // k bytes per LDS stage
constexpr int PITCH = BK + 16;     // padded LDS row (bytes)
constexpr int GROUP_M = 8;

template <int BIAS_DT>
__device__ __forceinline__ float load_bias(const void* b, int n) {
  if constexpr (BIAS_DT == DC_F32) return static_cast<const float*>(b)[n];
  else return h16_to_f32<BIAS_DT>(static_cast<const uint16_t*>(b)[n]);
}

// A float32 / 16-bit float element as its bits, and back to a float.
template <int DT>
__device__ __forceinline__ uint32_t raw_bits(const void* b, int n) {
  if constexpr (DT == DC_F32) return __float_as_uint(static_cast<const float*>(b)[n]);
  else return static_cast<const uint16_t*>(b)[n];
}
template <int DT>
__device__ __forceinline__ float from_bits(uint32_t v) {
  if constexpr (DT == DC_F32) return __uint_as_float(v);
  else return h16_to_f32<DT>(v);
}

template <int OUT_DT, int BIAS_DT>
__device__ __forceinline__ float epi(int acc, float sxm, float swn, const void* bias, int n) {
  float y = round_to<OUT_DT>(materialize((float)acc * (sxm * swn)));
  if constexpr (BIAS_DT != DC_NONE)
    y = round_to<OUT_DT>(materialize(y + round_to<OUT_DT>(load_bias<BIAS_DT>(bias, n))));
  return y;
}

// Same rounding with the bias already rounded to the output dtype (`b`).
template <int OUT_DT, bool HAS_BIAS>
__device__ __forceinline__ float epi_pre(int acc, float sxm, float swn, float b) {
  float y = round_to<OUT_DT>(materialize((float)acc * (sxm * swn)));
  if constexpr (HAS_BIAS) y = round_to<OUT_DT>(materialize(y + b));
  return y;
}

// 16-bit outputs two at a time, rounded as epi_pre rounds each (float32
// product; round to the output type; plus the rounded bias in float32; round
// again), with one packed conversion per rounding step.
template <int OUT_DT>
__device__ __forceinline__ uint32_t cvt_pair(float a, float b) {
  const v2f x = {a, b};
  if constexpr (OUT_DT == DC_BF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, v2bf));
  else return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, v2h));
}
template <int OUT_DT>
__device__ __forceinline__ float pair_lo(uint32_t pk) {
  if constexpr (OUT_DT == DC_BF16) return __uint_as_float(pk << 16);
  else return f16_to_f32(pk & 0xffffu);
}
template <int OUT_DT>
__device__ __forceinline__ float pair_hi(uint32_t pk) {
  if constexpr (OUT_DT == DC_BF16) return __uint_as_float(pk & 0xffff0000u);
  else return f16_to_f32(pk >> 16);
}
template <int OUT_DT, bool HAS_BIAS>
__device__ __forceinline__ uint32_t epi_pair(int a0, int a1, float sxm, float s0, float s1, float b0, float b1) {
  uint32_t pk = cvt_pair<OUT_DT>(materialize((float)a0 * (sxm * s0)), materialize((float)a1 * (sxm * s1)));
  if constexpr (HAS_BIAS)
    pk = cvt_pair<OUT_DT>(materialize(pair_lo<OUT_DT>(pk) + b0), materialize(pair_hi<OUT_DT>(pk) + b1));
  return pk;
}

// Gated residual on an output y (FLUX's x + gate * y, rounded as torch
// rounds its two ops): t = round(gate * y), out = round(res + t), each to the
// output type, with no contraction into an FMA.
template <int OUT_DT>
__device__ __forceinline__ float gated1(float y, float r, float g) {
  return round_to<OUT_DT>(materialize(r + round_to<OUT_DT>(materialize(g * y))));
}
// The same on two packed 16-bit outputs / residuals (one packed conversion
// per rounding step).
template <int OUT_DT>
__device__ __forceinline__ uint32_t gated_pair(uint32_t y2, uint32_t r2, float g0, float g1) {
  const uint32_t t2 = cvt_pair<OUT_DT>(materialize(g0 * pair_lo<OUT_DT>(y2)), materialize(g1 * pair_hi<OUT_DT>(y2)));
  return cvt_pair<OUT_DT>(materialize(pair_lo<OUT_DT>(r2) + pair_lo<OUT_DT>(t2)),
                          materialize(pair_hi<OUT_DT>(r2) + pair_hi<OUT_DT>(t2)));
}
// Eight packed 16-bit outputs (or four float32 ones) of one 16-byte chunk.
template <int OUT_DT>
__device__ __forceinline__ uint4 gated_chunk(uint4 y, uint4 r, const float* g) {
  if constexpr (OUT_DT == DC_F32) {
    return make_uint4(__float_as_uint(gated1<OUT_DT>(__uint_as_float(y.x), __uint_as_float(r.x), g[0])),
                      __float_as_uint(gated1<OUT_DT>(__uint_as_float(y.y), __uint_as_float(r.y), g[1])),
                      __float_as_uint(gated1<OUT_DT>(__uint_as_float(y.z), __uint_as_float(r.z), g[2])),
                      __float_as_uint(gated1<OUT_DT>(__uint_as_float(y.w), __uint_as_float(r.w), g[3])));
  } else {
    return make_uint4(gated_pair<OUT_DT>(y.x, r.x, g[0], g[1]), gated_pair<OUT_DT>(y.y, r.y, g[2], g[3]),
                      gated_pair<OUT_DT>(y.z, r.z, g[4], g[5]), gated_pair<OUT_DT>(y.w, r.w, g[6], g[7]));
  }
}

template <int OUT_DT>
__device__ __forceinline__ void store1(void* out, int64_t idx, float y) {
  if constexpr (OUT_DT == DC_F32) static_cast<float*>(out)[idx] = y;
  else static_cast<uint16_t*>(out)[idx] = (uint16_t)f32_to_h16<OUT_DT>(y);
}

// Tile configuration: WN x WM waves, each owning FN x FM MFMA blocks of 32 x 32.
// WN x WM waves, each FN x FM MFMA blocks of 32 x 32; RB register tiles of
// global loads in flight (tile kt + 1 + RB is fetched during iteration kt)
template <int WN_, int WM_, int FN_, int FM_, int RB_>
struct Tile {
  static constexpr int WN = WN_, WM = WM_, FN = FN_, FM = FM_, RB = RB_;
  static constexpr int NT = 64 * WN * WM;               // threads
  static constexpr int BN = 32 * WN * FN, BM = 32 * WM * FM;
  static constexpr int LDS = 2 * (BN + BM) * PITCH + (2 * BN + BM) * 4;
};

// Tile order: XCD-contiguous ranges of workgroups (the hardware deals them
// round-robin over the 8 XCDs), then GROUP_M m-tiles per sweep along n.

// Workgroup blockIdx.x's logical tile.
__device__ __forceinline__ int xcd_logical() {
  const int nwg = gridDim.x, wg = blockIdx.x;
  return (nwg % 8 == 0) ? (wg % 8) * (nwg / 8) + wg / 8 : wg;
}

// Origin of logical tile `logical` of a tiles_m x tiles_n grid: GROUP_M
// m-tiles per sweep along n.
__device__ __forceinline__ void tile_coords(int logical, int tiles_m, int tiles_n, int BM, int BN, int& m0, int& n0) {
  const int per_group = GROUP_M * tiles_n;
  const int grp = logical / per_group;
  const int first_m = grp * GROUP_M;
  const int gsize = min(tiles_m - first_m, GROUP_M);
  m0 = (first_m + (logical % per_group) % gsize) * BM;
  n0 = ((logical % per_group) / gsize) * BN;
}

__device__ __forceinline__ void tile_origin(const GemmArgs& p, int BM, int BN, int& m0, int& n0) {
  tile_coords(xcd_logical(), p.tiles_m, p.tiles_n, BM, BN, m0, n0);
}

// Grouped launch: the problem that owns this workgroup's logical tile, its
// fields copied into p (every index a constant: no dynamic indexing of the
// kernel arguments), and the tile's origin in that problem.
static_assert(DC_GEMM_MAX_GROUP == 4, "group_origin selects among 4 problems");
__device__ __forceinline__ void group_origin(GemmArgs& p, const GroupArgs& g, int BM, int BN, int& m0, int& n0) {
  const int logical = xcd_logical();
  const int k = (g.ngroup > 3 && logical >= g.first[3]) ? 3
              : (g.ngroup > 2 && logical >= g.first[2]) ? 2
              : (g.ngroup > 1 && logical >= g.first[1]) ? 1 : 0;
#define DC_SEL(f_) (k == 0 ? g.prob[0].f_ : k == 1 ? g.prob[1].f_ : k == 2 ? g.prob[2].f_ : g.prob[3].f_)
  p.a = DC_SEL(a); p.w = DC_SEL(w); p.sx = DC_SEL(sx); p.sw = DC_SEL(sw); p.bias = DC_SEL(bias);
  p.out = DC_SEL(out); p.lda = DC_SEL(lda); p.ldw = DC_SEL(ldw); p.ldo = DC_SEL(ldo);
  p.M = DC_SEL(M); p.tiles_m = DC_SEL(tiles_m); p.vec_out = DC_SEL(vec_out); p.vec16 = DC_SEL(vec16);
  p.res = DC_SEL(res); p.gate = DC_SEL(gate); p.ldr = DC_SEL(ldr);
  const int first = k == 0 ? g.first[0] : k == 1 ? g.first[1] : k == 2 ? g.first[2] : g.first[3];
#undef DC_SEL
  tile_coords(logical - first, p.tiles_m, p.tiles_n, BM, BN, m0, n0);
}

// Stores one workgroup tile from its MFMA accumulators (C^T layout): register
// r of acc[i][j] is output n = n0 + nb + 32 i + 8 (r / 4) + 4 hf + r % 4,
// m = m0 + mb + 32 j + l32. sw_l / b_l / sx_l are the tile's channel scales,
// rounded biases and row scales in LDS; each lane reads its row scales once
// and each group of 4 channel scales / biases once for all its rows.
// RES: the gated residual, with the tile's gate values in g_l (LDS).
template <int OUT_DT, int BIAS_DT, int FN, int FM, bool RES = false>
__device__ __forceinline__ void store_tile(const v16i (&acc)[FN][FM], const GemmArgs& p, int m0, int n0, int nb,
                                           int mb, int BM, int BN, const float* sw_l, const float* b_l,
                                           const float* sx_l, int hf, int l32, const float* g_l = nullptr) {
  constexpr bool HB = BIAS_DT != DC_NONE;
  const bool full = p.vec_out && m0 + BM <= p.M && n0 + BN <= p.N;
  float sxm[FM];
#pragma unroll
  for (int j = 0; j < FM; ++j) sxm[j] = OUT_DT != DC_I32 ? sx_l[mb + 32 * j + l32] : 0.0f;
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int nl = nb + 32 * i + 8 * g + 4 * hf, n = n0 + nl;
      const bool vec = full || (p.vec_out && n + 3 < p.N);
      float4 s4 = make_float4(0.f, 0.f, 0.f, 0.f), b4 = make_float4(0.f, 0.f, 0.f, 0.f);
      float4 g4 = make_float4(0.f, 0.f, 0.f, 0.f);
      if constexpr (OUT_DT != DC_I32) s4 = *reinterpret_cast<const float4*>(sw_l + nl);
      if constexpr (HB) b4 = *reinterpret_cast<const float4*>(b_l + nl);
      if constexpr (RES) g4 = *reinterpret_cast<const float4*>(g_l + nl);
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const int m = m0 + mb + 32 * j + l32;
        if (!full && m >= p.M) continue;
        const int64_t rbase = RES ? (int64_t)m * p.ldr + n : 0;
        const int64_t base = (int64_t)m * p.ldo + n;
        const int av[4] = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
        if constexpr (OUT_DT == DC_I32) {
          int* o = static_cast<int*>(p.out);
          if (vec) *reinterpret_cast<int4*>(o + base) = make_int4(av[0], av[1], av[2], av[3]);
          else for (int e = 0; e < 4 && n + e < p.N; ++e) o[base + e] = av[e];
        } else if constexpr (OUT_DT == DC_F32) {
          float y0 = epi_pre<OUT_DT, HB>(av[0], sxm[j], s4.x, b4.x);
          float y1 = epi_pre<OUT_DT, HB>(av[1], sxm[j], s4.y, b4.y);
          float y2 = epi_pre<OUT_DT, HB>(av[2], sxm[j], s4.z, b4.z);
          float y3 = epi_pre<OUT_DT, HB>(av[3], sxm[j], s4.w, b4.w);
          if constexpr (RES) {
            const float* r32 = static_cast<const float*>(p.res) + rbase;
            float4 r4 = make_float4(0.f, 0.f, 0.f, 0.f);
            if (vec) {
              r4 = *reinterpret_cast<const float4*>(r32);
            } else {
              if (n < p.N) r4.x = r32[0];
              if (n + 1 < p.N) r4.y = r32[1];
              if (n + 2 < p.N) r4.z = r32[2];
              if (n + 3 < p.N) r4.w = r32[3];
            }
            y0 = gated1<OUT_DT>(y0, r4.x, g4.x);
            y1 = gated1<OUT_DT>(y1, r4.y, g4.y);
            y2 = gated1<OUT_DT>(y2, r4.z, g4.z);
            y3 = gated1<OUT_DT>(y3, r4.w, g4.w);
          }
          if (vec) {
            *reinterpret_cast<float4*>(static_cast<float*>(p.out) + base) = make_float4(y0, y1, y2, y3);
          } else {
            const float yv[4] = {y0, y1, y2, y3};
            for (int e = 0; e < 4 && n + e < p.N; ++e) store1<OUT_DT>(p.out, base + e, yv[e]);
          }
        } else {
          uint32_t lo = epi_pair<OUT_DT, HB>(av[0], av[1], sxm[j], s4.x, s4.y, b4.x, b4.y);
          uint32_t hi = epi_pair<OUT_DT, HB>(av[2], av[3], sxm[j], s4.z, s4.w, b4.z, b4.w);
          if constexpr (RES) {
            const uint16_t* r16 = static_cast<const uint16_t*>(p.res) + rbase;
            uint32_t rlo, rhi;
            if (vec) {
              const uint2 rr = *reinterpret_cast<const uint2*>(r16);
              rlo = rr.x, rhi = rr.y;
            } else {
              uint32_t rv[4] = {0u, 0u, 0u, 0u};
              for (int e = 0; e < 4 && n + e < p.N; ++e) rv[e] = r16[e];
              rlo = rv[0] | (rv[1] << 16), rhi = rv[2] | (rv[3] << 16);
            }
            lo = gated_pair<OUT_DT>(lo, rlo, g4.x, g4.y);
            hi = gated_pair<OUT_DT>(hi, rhi, g4.z, g4.w);
          }
          uint16_t* o16 = static_cast<uint16_t*>(p.out);
          if (vec) {
            *reinterpret_cast<uint2*>(o16 + base) = make_uint2(lo, hi);
          } else {
            const uint32_t hv[4] = {lo & 0xffffu, lo >> 16, hi & 0xffffu, hi >> 16};
            for (int e = 0; e < 4 && n + e < p.N; ++e) o16[base + e] = (uint16_t)hv[e];
          }
        }
      }
    }
}

// This tile's epilogue vectors for thread t: output-channel scale, bias
// and gate (RES) of channel n0 + t (t < BN) and row scale of row m0 + t
// (t < BM), as loaded (16-bit values as their bits). Every tile shape has
// BN, BM <= its thread count, so one entry per thread covers them. They are
// loaded at the start of the tile, before its operand loads, and written to
// LDS (EpiRegs::stage) only once those have been waited for, so their memory
// latency runs under the operand loads' instead of ahead of it.
struct EpiRegs {
  uint32_t sw, b, sx, g;

  template <int OUT_DT, int BIAS_DT, bool RES = false>
  __device__ __forceinline__ static EpiRegs load(const GemmArgs& p, int m0, int n0, int BM, int BN, int t) {
    EpiRegs r{0u, 0u, 0u, 0u};
    if constexpr (OUT_DT != DC_I32) {
      const int n = min(n0 + t, p.N - 1);
      if (t < BN) {
        r.sw = __float_as_uint(p.sw[n]);
        if constexpr (BIAS_DT != DC_NONE) r.b = raw_bits<BIAS_DT>(p.bias, n);
        if constexpr (RES) r.g = raw_bits<OUT_DT>(p.gate, n);   // the gate is of the output dtype
      }
      if (t < BM) r.sx = __float_as_uint(p.sx[min(m0 + t, p.M - 1)]);
    }
    return r;
  }

  // Into the tile's LDS vectors: scales as loaded, the bias rounded to the
  // output dtype, the gate as a float.
  // The values pass an empty asm here first: without it the compiler moves
  // the bias rounding up to the load and waits for the load there.
  template <int OUT_DT, int BIAS_DT, bool RES = false>
  __device__ __forceinline__ void stage(int BM, int BN, int t, float* sw_l, float* b_l, float* sx_l,
                                        float* g_l = nullptr) const {
    if constexpr (OUT_DT != DC_I32) {
      uint32_t vsw = sw, vb = b, vsx = sx, vg = g;
      asm volatile("" : "+v"(vsw), "+v"(vb), "+v"(vsx), "+v"(vg));
      if (t < BN) {
        sw_l[t] = __uint_as_float(vsw);
        if constexpr (BIAS_DT != DC_NONE) b_l[t] = round_to<OUT_DT>(from_bits<BIAS_DT>(vb));
        if constexpr (RES) g_l[t] = from_bits<OUT_DT>(vg);
      }
      if (t < BM) sx_l[t] = __uint_as_float(vsx);
    }
  }
};

// Epilogue of one wave's full 128 (n) x 128 (m) block through LDS: the output
// values go to the wave's own 32 KB of LDS (`stage`, free after the main
// loop), row m at 128 * (output bytes) per row, 16-byte chunk c of row r at
// chunk c ^ (r % 16); then each row leaves as one contiguous run, 16 bytes per
// lane (4 rows per store instruction for 16-bit outputs, 2 for 32-bit). The
// MFMA layout would otherwise store 8 or 16 bytes into each of 32 rows per
// instruction. 32-bit outputs take two passes of 64 rows. A lane reads back
// what other lanes of its wave wrote: the wavefront fences and barrier
// between the two halves keep the compiler from moving LDS accesses across.
// RES: the gated residual. The residual chunks the lane stores go through a
// ring of RRING registers, loaded RRING stores ahead: the first RRING before
// the pass converts (they land meanwhile), each later one as its slot frees
// (a whole pass at once would spill). The lane's gate values come from g_l.
template <int OUT_DT, int BIAS_DT, bool RES = false>
__device__ __forceinline__ void store_tile_lds(const v16i (&acc)[4][4], const GemmArgs& p, int m0, int n0, int nb,
                                               int mb, const float* sw_l, const float* b_l, const float* sx_l, int hf,
                                               int l32, int lane, uint8_t* stage, const float* g_l = nullptr) {
  constexpr int OB = (OUT_DT == DC_F16 || OUT_DT == DC_BF16) ? 2 : 4;
  constexpr int ROWB = 128 * OB;   // staged row bytes
  constexpr int CH = ROWB / 16;    // 16-byte chunks per row
  constexpr int JP = 8 / OB;       // 32-row m blocks per pass
  constexpr int RPI = 64 / CH;     // rows per store instruction
  constexpr int NIT = 32 * JP / RPI;   // store instructions per pass
  constexpr int RRING = 8;             // residual chunks in flight per lane
  constexpr bool HB = BIAS_DT != DC_NONE;
  const int c = lane % CH;
  float sxm[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) sxm[j] = OUT_DT != DC_I32 ? sx_l[mb + 32 * j + l32] : 0.0f;
  float gv[RES ? 16 / OB : 1];
  if constexpr (RES) {
#pragma unroll
    for (int e = 0; e < 16 / OB; ++e) gv[e] = g_l[nb + (16 / OB) * c + e];
  }
#pragma unroll
  for (int j0 = 0; j0 < 4; j0 += JP) {
    uint4 rres[RES ? RRING : 1];
    const uint8_t* rrow = RES ? static_cast<const uint8_t*>(p.res) + (n0 + nb) * OB + 16 * c : nullptr;
    auto rload = [&](int k) __attribute__((always_inline)) {
      return *reinterpret_cast<const uint4*>(rrow + (int64_t)(m0 + mb + 32 * j0 + RPI * k + lane / CH) * p.ldr * OB);
    };
    if constexpr (RES) {
#pragma unroll
      for (int k = 0; k < RRING; ++k) rres[k] = rload(k);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int nl = nb + 32 * i + 8 * g + 4 * hf;
        float4 s4 = make_float4(0.f, 0.f, 0.f, 0.f), b4 = make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (OUT_DT != DC_I32) s4 = *reinterpret_cast<const float4*>(sw_l + nl);
        if constexpr (HB) b4 = *reinterpret_cast<const float4*>(b_l + nl);
#pragma unroll
        for (int jj = 0; jj < JP; ++jj) {
          const int j = j0 + jj, r = 32 * jj + l32;
          uint8_t* row = stage + r * ROWB;
          const int av[4] = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
          if constexpr (OUT_DT == DC_I32) {
            const int c = 8 * i + 2 * g + hf;
            *reinterpret_cast<int4*>(row + 16 * (c ^ (r & 15))) = make_int4(av[0], av[1], av[2], av[3]);
          } else if constexpr (OUT_DT == DC_F32) {
            const int c = 8 * i + 2 * g + hf;
            const float y0 = epi_pre<OUT_DT, HB>(av[0], sxm[j], s4.x, b4.x);
            const float y1 = epi_pre<OUT_DT, HB>(av[1], sxm[j], s4.y, b4.y);
            const float y2 = epi_pre<OUT_DT, HB>(av[2], sxm[j], s4.z, b4.z);
            const float y3 = epi_pre<OUT_DT, HB>(av[3], sxm[j], s4.w, b4.w);
            *reinterpret_cast<float4*>(row + 16 * (c ^ (r & 15))) = make_float4(y0, y1, y2, y3);
          } else {
            const int c = 4 * i + g;
            const uint32_t lo = epi_pair<OUT_DT, HB>(av[0], av[1], sxm[j], s4.x, s4.y, b4.x, b4.y);
            const uint32_t hi = epi_pair<OUT_DT, HB>(av[2], av[3], sxm[j], s4.z, s4.w, b4.z, b4.w);
            *reinterpret_cast<uint2*>(row + 16 * (c ^ (r & 15)) + 8 * hf) = make_uint2(lo, hi);
          }
        }
      }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int k = 0; k < NIT; ++k) {
      const int r = RPI * k + lane / CH;
      uint4 v = *reinterpret_cast<const uint4*>(stage + r * ROWB + 16 * (c ^ (r & 15)));
      if constexpr (RES) {
        const uint4 rk = rres[k % RRING];
        if (k + RRING < NIT) rres[k % RRING] = rload(k + RRING);
        v = gated_chunk<OUT_DT>(v, rk, gv);
      }
      const int64_t m = m0 + mb + 32 * j0 + r;
      uint8_t* dst = static_cast<uint8_t*>(p.out) + (m * p.ldo + n0 + nb) * OB + 16 * c;
      *reinterpret_cast<uint4*>(dst) = v;
    }
    if constexpr (JP < 4) {
      // the next pass overwrites what this one read back
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
}

// Epilogue of one wave's full (32 FN) n x (32 FM) m block through LDS, for the
// register-staged kernel: the wave's outputs go to its own WAVE_BYTES of the
// LDS stages (free after the main loop), row m at a pitch of its bytes plus
// 16 (the padding spreads a 16-byte write of 16 consecutive rows over all
// banks), JP 32-row m blocks per pass; then each row leaves as one contiguous
// run, 16 bytes per lane. Stored from the MFMA layout instead, one
// instruction writes 16 or 32 bytes into each of 32 rows. Same rounding as
// store_tile. A lane reads back what other lanes of its wave wrote: the
// wavefront fences and barrier keep the compiler from moving LDS accesses
// across.
template <int OUT_DT, int BIAS_DT, int FN, int FM, int WAVE_BYTES>
__device__ __forceinline__ void store_tile_staged(const v16i (&acc)[FN][FM], const GemmArgs& p, int m0, int n0, int nb,
                                                  int mb, const float* sw_l, const float* b_l, const float* sx_l,
                                                  int hf, int l32, int lane, uint8_t* stage) {
  constexpr int OB = (OUT_DT == DC_F16 || OUT_DT == DC_BF16) ? 2 : 4;
  constexpr int ROWB = 32 * FN * OB;   // output row bytes of the block
  constexpr int RP = ROWB + 16;        // staged row pitch
  constexpr int CH = ROWB / 16;        // 16-byte chunks per row
  constexpr int JP = (FM % 2 == 0 && 64 * RP <= WAVE_BYTES) ? 2 : 1;   // 32-row m blocks per pass
  constexpr int NIT = 32 * JP * CH / 64;                              // store instructions per pass
  static_assert(32 * RP <= WAVE_BYTES, "one 32-row block must fit the wave's LDS share");
  static_assert((32 * JP * CH) % 64 == 0, "a pass must be whole store instructions");
  constexpr bool HB = BIAS_DT != DC_NONE;
  float sxm[FM];
#pragma unroll
  for (int j = 0; j < FM; ++j) sxm[j] = OUT_DT != DC_I32 ? sx_l[mb + 32 * j + l32] : 0.0f;
#pragma unroll
  for (int j0 = 0; j0 < FM; j0 += JP) {
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int nl = nb + 32 * i + 8 * g + 4 * hf;
        float4 s4 = make_float4(0.f, 0.f, 0.f, 0.f), b4 = make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (OUT_DT != DC_I32) s4 = *reinterpret_cast<const float4*>(sw_l + nl);
        if constexpr (HB) b4 = *reinterpret_cast<const float4*>(b_l + nl);
#pragma unroll
        for (int jj = 0; jj < JP; ++jj) {
          const int j = j0 + jj;
          uint8_t* row = stage + (32 * jj + l32) * RP;
          const int av[4] = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
          if constexpr (OUT_DT == DC_I32) {
            *reinterpret_cast<int4*>(row + 16 * (8 * i + 2 * g + hf)) = make_int4(av[0], av[1], av[2], av[3]);
          } else if constexpr (OUT_DT == DC_F32) {
            const float y0 = epi_pre<OUT_DT, HB>(av[0], sxm[j], s4.x, b4.x);
            const float y1 = epi_pre<OUT_DT, HB>(av[1], sxm[j], s4.y, b4.y);
            const float y2 = epi_pre<OUT_DT, HB>(av[2], sxm[j], s4.z, b4.z);
            const float y3 = epi_pre<OUT_DT, HB>(av[3], sxm[j], s4.w, b4.w);
            *reinterpret_cast<float4*>(row + 16 * (8 * i + 2 * g + hf)) = make_float4(y0, y1, y2, y3);
          } else {
            const uint32_t lo = epi_pair<OUT_DT, HB>(av[0], av[1], sxm[j], s4.x, s4.y, b4.x, b4.y);
            const uint32_t hi = epi_pair<OUT_DT, HB>(av[2], av[3], sxm[j], s4.z, s4.w, b4.z, b4.w);
            *reinterpret_cast<uint2*>(row + 16 * (4 * i + g) + 8 * hf) = make_uint2(lo, hi);
          }
        }
      }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int k = 0; k < NIT; ++k) {
      const int idx = 64 * k + lane, r = idx / CH, c = idx % CH;
      const uint4 v = *reinterpret_cast<const uint4*>(stage + r * RP + 16 * c);
      const int64_t m = m0 + mb + 32 * j0 + r;
      *reinterpret_cast<uint4*>(static_cast<uint8_t*>(p.out) + (m * p.ldo + n0 + nb) * OB + 16 * c) = v;
    }
    if (j0 + JP < FM) {
      // the next pass overwrites what this one read back
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
}

template <class T, int OUT_DT, int BIAS_DT>
__global__ void __launch_bounds__(T::NT, 1) w8a8_gemm_kernel(GemmArgs p) {
  constexpr int FN = T::FN, FM = T::FM, NT = T::NT;
  if constexpr (OUT_DT == DC_I32) {
    if (p.ksplit > 1) {
      const int k0 = (int)blockIdx.y * p.kslice;
      p.a += k0;
      p.w += k0;
      p.K = min(p.kslice, p.K - k0);
      p.out = static_cast<int32_t*>(p.out) + (int64_t)blockIdx.y * p.split_stride;
    }
  }
  constexpr int BN = T::BN, BM = T::BM;
  constexpr int CPR = BK / 16;                    // 16-byte chunks per row
  constexpr int NWL = BN * CPR / NT, NAL = BM * CPR / NT;
  static_assert(BN * CPR % NT == 0 && BM * CPR % NT == 0, "tile must split evenly over the threads");
  static_assert(BN <= NT && BM <= NT, "EpiRegs holds one epilogue-vector entry per thread");
  constexpr int STAGE = (BN + BM) * PITCH;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int l32 = lane & 31, hf = lane >> 5;

  int m0, n0;
  tile_origin(p, BM, BN, m0, n0);

  const int wn = wv % T::WN, wm = wv / T::WN;
  // per-lane fragment bases: row (wave base + l32), byte 16 hf; + 32 i rows, + 32 ks bytes
  const int wfrag = (wn * 32 * FN + l32) * PITCH + 16 * hf;
  const int afrag = BN * PITCH + (wm * 32 * FM + l32) * PITCH + 16 * hf;

  v16i acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = v16i{0};

  uint4 wst[T::RB][NWL], ast[T::RB][NAL];   // register tiles in flight
  v4i wf[2][FN], af[2][FM];
  const int nk = (p.K + BK - 1) / BK;

  // Row indices are clamped into range (rows past M or N only feed outputs that
  // are never stored) and chunks past K are zeroed by a mask when they are
  // stored to LDS, so the loads carry no branches and no waits.
  const int64_t kmax = p.K - 16;
#define GEMM_LOAD(buf_, kt_)                                                                             \
  {                                                                                                      \
    const int k0_ = (kt_) * BK;                                                                          \
    static_for<NWL>([&](auto u_) {                                                                       \
      constexpr int u = decltype(u_)::value;                                                             \
      const int ci = t + u * NT, r = ci / CPR, c = ci % CPR;                                             \
      const int n = min(n0 + r, p.N - 1), k = k0_ + 16 * c;                                              \
      wst[buf_][u] = *reinterpret_cast<const uint4*>(p.w + (int64_t)n * p.ldw + min((int64_t)k, kmax));  \
    });                                                                                                  \
    static_for<NAL>([&](auto u_) {                                                                       \
      constexpr int u = decltype(u_)::value;                                                             \
      const int ci = t + u * NT, r = ci / CPR, c = ci % CPR;                                             \
      const int m = min(m0 + r, p.M - 1), k = k0_ + 16 * c;                                              \
      ast[buf_][u] = *reinterpret_cast<const uint4*>(p.a + (int64_t)m * p.lda + min((int64_t)k, kmax));  \
    });                                                                                                  \
  }
#define GEMM_STORE(buf_, stage_, kt_)                                                                    \
  {                                                                                                      \
    uint8_t* base_ = smem + (stage_) * STAGE;                                                            \
    static_for<NWL>([&](auto u_) {                                                                       \
      constexpr int u = decltype(u_)::value;                                                             \
      const int ci = t + u * NT, r = ci / CPR, c = ci % CPR;                                             \
      const uint32_t km_ = (kt_) * BK + 16 * c < p.K ? ~0u : 0u;                                         \
      const uint4 v_ = wst[buf_][u];                                                                     \
      *reinterpret_cast<uint4*>(base_ + r * PITCH + c * 16) =                                            \
          make_uint4(v_.x & km_, v_.y & km_, v_.z & km_, v_.w & km_);                                    \
    });                                                                                                  \
    static_for<NAL>([&](auto u_) {                                                                       \
      constexpr int u = decltype(u_)::value;                                                             \
      const int ci = t + u * NT, r = ci / CPR, c = ci % CPR;                                             \
      const uint32_t km_ = (kt_) * BK + 16 * c < p.K ? ~0u : 0u;                                         \
      const uint4 v_ = ast[buf_][u];                                                                     \
      *reinterpret_cast<uint4*>(base_ + BN * PITCH + r * PITCH + c * 16) =                               \
          make_uint4(v_.x & km_, v_.y & km_, v_.z & km_, v_.w & km_);                                    \
    });                                                                                                  \
  }
#define GEMM_FRAGS(buf_, stage_, ks_)                                                                    \
  {                                                                                                      \
    const uint8_t* base_ = smem + (stage_) * STAGE + 32 * (ks_);                                         \
    _Pragma("unroll") for (int i = 0; i < FN; ++i)                                                       \
        wf[buf_][i] = *reinterpret_cast<const v4i*>(base_ + wfrag + 32 * i * PITCH);                     \
    _Pragma("unroll") for (int j = 0; j < FM; ++j)                                                       \
        af[buf_][j] = *reinterpret_cast<const v4i*>(base_ + afrag + 32 * j * PITCH);                     \
  }
#define GEMM_MFMAS(buf_)                                                                                 \
  _Pragma("unroll") for (int i = 0; i < FN; ++i)                                                         \
  _Pragma("unroll") for (int j = 0; j < FM; ++j)                                                         \
      acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[buf_][i], af[buf_][j], acc[i][j], 0, 0, 0);
// scheduler hints: `n` MFMAs, each followed by `per` instructions of class `mask`
#define SCHED_INTERLEAVE(n_, mask_, per_)                                                                \
  _Pragma("unroll") for (int z = 0; z < (n_); ++z) {                                                     \
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                                   \
    __builtin_amdgcn_sched_group_barrier((mask_), (per_), 0);                                            \
  }                                                                                                      \
  if constexpr ((n_) == 0) __builtin_amdgcn_sched_group_barrier((mask_), 64, 0);

  constexpr int NF = FN + FM;                  // fragment reads per k-step
  constexpr int NMF = FN * FM;                 // MFMAs per k-step
  constexpr int NST = NWL + NAL;               // 16-byte stores / loads per thread per tile
  constexpr int NSLOT = NMF > NF ? NMF - NF : 0;          // MFMAs left for stores / loads
  constexpr int PER = NSLOT ? (NST + NSLOT - 1) / NSLOT : 1;
  // this tile's output-channel scales, biases (rounded to the output dtype)
  // and row scales, staged in LDS for the epilogue
  float* sw_l = reinterpret_cast<float*>(smem + 2 * STAGE);
  float* b_l = sw_l + BN;
  float* sx_l = b_l + BN;
  const EpiRegs ev = EpiRegs::load<OUT_DT, BIAS_DT>(p, m0, n0, BM, BN, t);
  GEMM_LOAD(0, 0);
  GEMM_STORE(0, 0, 0);
  ev.stage<OUT_DT, BIAS_DT>(BM, BN, t, sw_l, b_l, sx_l);   // loaded before tile 0, so already here
  static_for<T::RB>([&](auto i_) {
    constexpr int i = decltype(i_)::value + 1;
    GEMM_LOAD(i % T::RB, i);
  });
  __syncthreads();
  GEMM_FRAGS(0, 0, 0);
  // Each k-step is its own scheduling region: its MFMAs consume fragments read
  // one k-step earlier while it issues the reads for the next one. Register
  // tile (kt + 1) % RB holds tile kt + 1 (fetched RB iterations earlier): it
  // goes to LDS stage cur ^ 1 in k-step 0 and is refilled with tile kt + 1 + RB
  // in k-step 1. Barrier A (all waves stored tile kt + 1) lets k-step 3 prefetch
  // tile kt + 1's first fragments; barrier B (all waves done reading stage cur)
  // guards the next iteration's store into it. Two iterations per trip keep the
  // register tile indices constant.
#define GEMM_ITER(kt_, rb_)                                                                              \
  {                                                                                                      \
    const int cur = (kt_) & 1;                                                                           \
    GEMM_FRAGS(1, cur, 1);                                                                               \
    GEMM_MFMAS(0);                                                                                       \
    GEMM_STORE(rb_, cur ^ 1, (kt_) + 1);                                                                 \
    SCHED_INTERLEAVE(NF, 0x100, 1);                                                                      \
    SCHED_INTERLEAVE(NSLOT, 0x200, PER);                                                                 \
    __builtin_amdgcn_sched_barrier(0);                                                                   \
    GEMM_FRAGS(0, cur, 2);                                                                               \
    GEMM_MFMAS(1);                                                                                       \
    GEMM_LOAD(rb_, (kt_) + 1 + T::RB);                                                                   \
    SCHED_INTERLEAVE(NF, 0x100, 1);                                                                      \
    SCHED_INTERLEAVE(NSLOT, 0x020, PER);                                                                 \
    __builtin_amdgcn_sched_barrier(0);                                                                   \
    GEMM_FRAGS(1, cur, 3);                                                                               \
    GEMM_MFMAS(0);                                                                                       \
    SCHED_INTERLEAVE(NF, 0x100, 1);                                                                      \
    __builtin_amdgcn_sched_barrier(0);                                                                   \
    __syncthreads();   /* A */                                                                           \
    GEMM_FRAGS(0, cur ^ 1, 0);                                                                           \
    GEMM_MFMAS(1);                                                                                       \
    SCHED_INTERLEAVE(NF, 0x100, 1);                                                                      \
    __builtin_amdgcn_sched_barrier(0);                                                                   \
    __syncthreads();   /* B */                                                                           \
  }
  int kt = 0;
  for (; kt + 1 < nk; kt += 2) {
    GEMM_ITER(kt, 1 % T::RB);
    GEMM_ITER(kt + 1, 0);
  }
  if (kt < nk) GEMM_ITER(kt, 1 % T::RB);
#undef GEMM_ITER
#undef SCHED_INTERLEAVE
#undef GEMM_MFMAS
#undef GEMM_LOAD
#undef GEMM_STORE
#undef GEMM_FRAGS

  // epilogue: acc[i][j] register r -> n = n0 + nb + 32 i + 8 (r / 4) + 4 hf + r % 4, m = m0 + mb + 32 j + l32;
  // whole tiles through the (now free) LDS stages, each wave in its own share
  constexpr int WAVE_BYTES = 2 * STAGE / (T::WN * T::WM) / 16 * 16;
  if (p.vec16 && m0 + BM <= p.M && n0 + BN <= p.N)
    store_tile_staged<OUT_DT, BIAS_DT, FN, FM, WAVE_BYTES>(acc, p, m0, n0, wn * 32 * FN, wm * 32 * FM, sw_l, b_l,
                                                           sx_l, hf, l32, lane, smem + wv * WAVE_BYTES);
  else
    store_tile<OUT_DT, BIAS_DT, FN, FM>(acc, p, m0, n0, wn * 32 * FN, wm * 32 * FM, BM, BN, sw_l, b_l, sx_l, hf, l32);
}

// ---------------------------------------------------------------- DMA-fed kernel
//
// 256 x 256 tiles on 4 waves (2 along n x 2 along m, each 128 x 128 = 4 x 4
// MFMA blocks, accumulators in AGPRs, one wave per SIMD). Operands go from
// global memory straight into LDS (global_load_lds_dwordx4: lane i of a wave
// writes bytes 16 i .. 16 i + 15 after the wave's base) through 4 stages of 64
// k-bytes, up to 4 stages ahead of the MFMAs, so no registers stage them. A stage is
// W [256 rows x 64 B] then A [256 rows x 64 B], unpadded; the 16-byte chunk c
// of row r sits at chunk c ^ ((r / 4) % 4), which spreads the 16 rows a
// fragment read serves per cycle over all banks. One barrier per stage, half
// way through it: every wave has waited for its own loads of the next stage
// (vmcnt) and for its own fragment reads of the current one (lgkmcnt), so
// after the barrier the next stage is complete and the current stage's buffer
// is free for the loads 4 stages ahead.
// Needs K % 256 == 0 (whole stages, 4 per trip of the unrolled loop) and
// 256 * ldw, 256 * lda below 2^31.
constexpr int DBK = 64;                      // k bytes per stage
constexpr int DSTAGE = (256 + 256) * DBK;    // 32 KB
constexpr int DMA_LOADS_PER_STAGE = 8;       // per wave: 4 KB of W + 4 KB of A

typedef __attribute__((address_space(3))) void* lds_void_ptr;

// vmcnt(n) with the other counters left unconstrained, and vmcnt(n) together
// with lgkmcnt(0) (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8)
#define DC_WAIT_VMCNT(n_) __builtin_amdgcn_s_waitcnt(((n_) & 15) | (((n_) >> 4) << 14) | (7 << 4) | (15 << 8))
#define DC_WAIT_VMCNT_LGKM0(n_) __builtin_amdgcn_s_waitcnt(((n_) & 15) | (((n_) >> 4) << 14) | (7 << 4))

// RES: with the gated residual of dc_w8a8_gemm_grouped_gated.
template <int OUT_DT, int BIAS_DT, bool RES = false>
__global__ void __launch_bounds__(256, 1) w8a8_gemm_dma_kernel(GemmArgs p, GroupArgs g) {
  constexpr int BN = 256, BM = 256, FN = 4, FM = 4;
  __shared__ __attribute__((aligned(1024))) uint8_t st0[DSTAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t st1[DSTAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t st2[DSTAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t st3[DSTAGE];
  __shared__ __attribute__((aligned(16))) float epi_v[(RES ? 3 : 2) * BN + BM];

  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int l32 = lane & 31, hf = lane >> 5;
  const int wn = w & 1, wm = w >> 1;
  int m0, n0;
  if (g.ngroup > 0) group_origin(p, g, BM, BN, m0, n0);
  else tile_origin(p, BM, BN, m0, n0);

  float* sw_l = epi_v;
  float* b_l = epi_v + BN;
  float* sx_l = epi_v + 2 * BN;
  float* g_l = RES ? epi_v + 2 * BN + BM : nullptr;
  // issued ahead of the operand loads; staged in LDS after the main loop
  const EpiRegs ev = EpiRegs::load<OUT_DT, BIAS_DT, RES>(p, m0, n0, BM, BN, t);

  // DMA sources: wave w loads 1 KB blocks j = w + 4 u (rows 16 j .. 16 j + 15)
  // of W and of A; lane i covers row 16 j + i / 4, logical chunk
  // (i % 4) ^ ((i / 16) % 4) (its physical chunk is i % 4).
  // (byte offsets from the tile's first W / A row; rows past N / M are clamped)
  const int drow = lane >> 2, dchunk = (lane & 3) ^ ((lane >> 4) & 3);
  const int8_t* wtile = p.w + (int64_t)n0 * p.ldw;
  const int8_t* atile = p.a + (int64_t)m0 * p.lda;
  uint32_t woff[4], aoff[4];   // unsigned: a scalar base plus a 32-bit lane offset
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int r = 16 * (w + 4 * u) + drow;
    woff[u] = (uint32_t)((min(n0 + r, p.N - 1) - n0) * (int)p.ldw + 16 * dchunk);
    aoff[u] = (uint32_t)((min(m0 + r, p.M - 1) - m0) * (int)p.lda + 16 * dchunk);
  }
  const int nk = p.K / DBK;   // a multiple of 4
  // stage kt's loads; stages past the end re-read the last one (kept in bounds;
  // their data is never used)
#define DMA_STAGE(buf_, kt_)                                                                             \
  {                                                                                                      \
    const int k0_ = min((kt_), nk - 1) * DBK;                                                            \
    _Pragma("unroll") for (int u = 0; u < 4; ++u)                                                        \
        __builtin_amdgcn_global_load_lds((wtile + k0_) + woff[u], (lds_void_ptr)((buf_) + 1024 * (w + 4 * u)), 16, 0, 0); \
    _Pragma("unroll") for (int u = 0; u < 4; ++u)                                                        \
        __builtin_amdgcn_global_load_lds((atile + k0_) + aoff[u], (lds_void_ptr)((buf_) + 16384 + 1024 * (w + 4 * u)), 16, 0, 0); \
  }

  // fragment reads: W rows wn*128 + 32 i + l32, A rows wm*128 + 32 j + l32; k-step
  // ks reads logical chunk 2 ks + hf, physical (2 ks + hf) ^ ((l32 / 4) % 4)
  const int swz = (l32 >> 2) & 3;
  const int wrow = (wn * 128 + l32) * DBK, arow = 16384 + (wm * 128 + l32) * DBK;
  const int kc0 = 16 * (hf ^ swz), kc1 = 16 * ((2 + hf) ^ swz);
  v16i acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = v16i{0};
  v4i wf[2][FN], af[2][FM];
#define DMA_FRAGS(b_, buf_, kc_)                                                                         \
  {                                                                                                      \
    _Pragma("unroll") for (int i = 0; i < FN; ++i)                                                       \
        wf[b_][i] = *reinterpret_cast<const v4i*>((buf_) + wrow + 2048 * i + (kc_));                     \
    _Pragma("unroll") for (int j = 0; j < FM; ++j)                                                       \
        af[b_][j] = *reinterpret_cast<const v4i*>((buf_) + arow + 2048 * j + (kc_));                     \
  }
#define DMA_MFMAS(b_)                                                                                    \
  _Pragma("unroll") for (int i = 0; i < FN; ++i)                                                         \
  _Pragma("unroll") for (int j = 0; j < FM; ++j)                                                         \
      acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[b_][i], af[b_][j], acc[i][j], 0, 0, 0);

  DMA_STAGE(st0, 0);
  DMA_STAGE(st1, 1);
  DMA_STAGE(st2, 2);
  DMA_STAGE(st3, 3);
  DC_WAIT_VMCNT(3 * DMA_LOADS_PER_STAGE);
  __builtin_amdgcn_s_barrier();
  DMA_FRAGS(0, st0, kc0);

  // Iteration kt (stage buffer cur = kt % 4): k-step 0 runs on fragments read
  // earlier while k-step 1's are read from cur; then the wave waits for its
  // loads of stage kt + 1 and for its reads of cur, the barrier makes stage
  // kt + 1 complete and cur free, the loads of stage kt + 4 go into cur, and
  // k-step 1 runs while the first fragments of stage kt + 1 are read.
#define DMA_ITER(kt_, cur_, nxt_)                                                                        \
  {                                                                                                      \
    DMA_FRAGS(1, cur_, kc1);                                                                             \
    DMA_MFMAS(0);                                                                                        \
    /* one MFMA first: its wait covers only the fragments it uses */                                     \
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                                   \
    _Pragma("unroll") for (int z = 0; z < 8; ++z) {                                                      \
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                                 \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                                 \
    }                                                                                                    \
    __builtin_amdgcn_sched_group_barrier(0x008, 7, 0);                                                   \
    __builtin_amdgcn_sched_barrier(0);                                                                   \
    DC_WAIT_VMCNT_LGKM0(2 * DMA_LOADS_PER_STAGE);                                                        \
    __builtin_amdgcn_s_barrier();                                                                        \
    __builtin_amdgcn_sched_barrier(0);                                                                   \
    DMA_STAGE(cur_, (kt_) + 4);                                                                          \
    DMA_FRAGS(0, nxt_, kc0);                                                                             \
    DMA_MFMAS(1);                                                                                        \
    /* the next fragment reads with the first 8 MFMAs (they return during the  \
       last 8, so the next iteration's first MFMA does not wait on them), the  \
       stage's loads with the last 8 */                                                                  \
    _Pragma("unroll") for (int z = 0; z < 8; ++z) {                                                      \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                                 \
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                                 \
    }                                                                                                    \
    _Pragma("unroll") for (int z = 0; z < 8; ++z) {                                                      \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                                 \
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                                                 \
    }                                                                                                    \
    __builtin_amdgcn_sched_barrier(0);                                                                   \
  }
  for (int kt = 0; kt < nk; kt += 4) {
    DMA_ITER(kt, st0, st1);
    DMA_ITER(kt + 1, st1, st2);
    DMA_ITER(kt + 2, st2, st3);
    DMA_ITER(kt + 3, st3, st0);
  }
#undef DMA_ITER
#undef DMA_MFMAS
#undef DMA_FRAGS
#undef DMA_STAGE
  // no load may still be writing this workgroup's LDS when it ends
  DC_WAIT_VMCNT(0);
  ev.stage<OUT_DT, BIAS_DT, RES>(BM, BN, t, sw_l, b_l, sx_l, g_l);
  __syncthreads();   // the epilogue vectors are in LDS; every wave is done reading the stage buffers

  if (p.vec16 && m0 + BM <= p.M && n0 + BN <= p.N) {
    uint8_t* stg = w == 0 ? st0 : (w == 1 ? st1 : (w == 2 ? st2 : st3));
    store_tile_lds<OUT_DT, BIAS_DT, RES>(acc, p, m0, n0, wn * 128, wm * 128, sw_l, b_l, sx_l, hf, l32, lane, stg,
                                         g_l);
  } else {
    store_tile<OUT_DT, BIAS_DT, FN, FM, RES>(acc, p, m0, n0, wn * 32 * FN, wm * 32 * FM, BM, BN, sw_l, b_l, sx_l,
                                             hf, l32, g_l);
  }
}

#undef DC_WAIT_VMCNT
#undef DC_WAIT_VMCNT_LGKM0

// Rescale pass over an int32 accumulator (dc_rescale), or over the sum of
// nsplit split-K partials split_stride apart (exact in int32): one thread
// per 4 outputs.
template <int OUT_DT, int BIAS_DT>
__global__ void __launch_bounds__(256) rescale_kernel(const int32_t* __restrict__ acc, int64_t lda,
                                                      const float* __restrict__ sx, const float* __restrict__ sw,
                                                      const void* __restrict__ bias, void* __restrict__ out,
                                                      int64_t ldo, int M, int N, int nsplit, int64_t split_stride) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int n4 = (N + 3) / 4;
  const int64_t m = idx / n4;
  const int n = (int)(idx % n4) * 4;
  if (m >= M) return;
  const float sxm = sx[m];
  for (int e = 0; e < 4 && n + e < N; ++e) {
    int32_t a = acc[m * lda + n + e];
    for (int s = 1; s < nsplit; ++s) a += acc[s * split_stride + m * lda + n + e];
    store1<OUT_DT>(out, m * ldo + n + e, epi<OUT_DT, BIAS_DT>(a, sxm, sw[n + e], bias, n + e));
  }
}

// The same pass four outputs at a time with 16-byte partial loads and one
// 8- or 16-byte store, when N, lda, ldo and split_stride are multiples of 4
// and acc and out are aligned to match (the split-K workspace always is).
// Each output is rounded by the same epi() as above.
template <int OUT_DT, int BIAS_DT>
__global__ void __launch_bounds__(256) rescale_vec_kernel(const int32_t* __restrict__ acc, int64_t lda,
                                                          const float* __restrict__ sx, const float* __restrict__ sw,
                                                          const void* __restrict__ bias, void* __restrict__ out,
                                                          int64_t ldo, int M, int N, int nsplit,
                                                          int64_t split_stride) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int n4 = N / 4;
  const int64_t m = idx / n4;
  const int n = (int)(idx % n4) * 4;
  if (m >= M) return;
  const int4* src = reinterpret_cast<const int4*>(acc + m * lda + n);
  int4 a = src[0];
  for (int s = 1; s < nsplit; ++s) {
    const int4 b = src[s * (split_stride / 4)];
    a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
  }
  const float sxm = sx[m];
  const float4 s4 = *reinterpret_cast<const float4*>(sw + n);
  const float y0 = epi<OUT_DT, BIAS_DT>(a.x, sxm, s4.x, bias, n);
  const float y1 = epi<OUT_DT, BIAS_DT>(a.y, sxm, s4.y, bias, n + 1);
  const float y2 = epi<OUT_DT, BIAS_DT>(a.z, sxm, s4.z, bias, n + 2);
  const float y3 = epi<OUT_DT, BIAS_DT>(a.w, sxm, s4.w, bias, n + 3);
  if constexpr (OUT_DT == DC_F32) {
    *reinterpret_cast<float4*>(static_cast<float*>(out) + m * ldo + n) = make_float4(y0, y1, y2, y3);
  } else {
    const uint32_t lo = f32_to_h16<OUT_DT>(y0) | (f32_to_h16<OUT_DT>(y1) << 16);
    const uint32_t hi = f32_to_h16<OUT_DT>(y2) | (f32_to_h16<OUT_DT>(y3) << 16);
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + m * ldo + n) = make_uint2(lo, hi);
  }
}

template <class T, int OUT_DT, int BIAS_DT>
static int launch_gemm(GemmArgs p, hipStream_t st) {
  p.tiles_n = (p.N + T::BN - 1) / T::BN;
  p.tiles_m = (p.M + T::BM - 1) / T::BM;
  const int64_t tiles = (int64_t)p.tiles_n * p.tiles_m;
  if (tiles > 0x7fffffff) return fail(DC_EINVAL, "dc_w8a8_gemm: problem too large");
  // the LDS attribute, set once per instantiation and device; threads that
  // race on a first call each set it (the call is idempotent)
  static std::atomic<bool> attr_set[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (!attr_set[dev].load(std::memory_order_acquire)) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&w8a8_gemm_kernel<T, OUT_DT, BIAS_DT>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, T::LDS);
    if (e != hipSuccess) {
      set_error("w8a8_gemm_kernel: cannot reserve %d bytes of LDS: %s", T::LDS, hipGetErrorString(e));
      return DC_EHIP;
    }
    attr_set[dev].store(true, std::memory_order_release);
  }
  const unsigned ks = p.ksplit > 1 ? (unsigned)p.ksplit : 1u;
  hipLaunchKernelGGL((w8a8_gemm_kernel<T, OUT_DT, BIAS_DT>), dim3((unsigned)tiles, ks), dim3(T::NT), T::LDS, st, p);
  return launch_status("w8a8_gemm_kernel");
}

template <int OUT_DT, int BIAS_DT>
static int launch_gemm_dma(GemmArgs p, hipStream_t st) {
  p.tiles_n = (p.N + 255) / 256;
  p.tiles_m = (p.M + 255) / 256;
  const int64_t tiles = (int64_t)p.tiles_n * p.tiles_m;
  if (tiles > 0x7fffffff) return fail(DC_EINVAL, "dc_w8a8_gemm: problem too large");
  hipLaunchKernelGGL((w8a8_gemm_dma_kernel<OUT_DT, BIAS_DT>), dim3((unsigned)tiles), dim3(256), 0, st, p, GroupArgs{});
  return launch_status("w8a8_gemm_dma_kernel");
}

// Grouped launch: g.first[g.ngroup] tiles in all (p holds N, K, tiles_n).
template <int OUT_DT, int BIAS_DT, bool RES = false>
static int launch_gemm_dma_group(GemmArgs p, const GroupArgs& g, hipStream_t st) {
  hipLaunchKernelGGL((w8a8_gemm_dma_kernel<OUT_DT, BIAS_DT, RES>), dim3((unsigned)g.first[g.ngroup]), dim3(256), 0, st,
                     p, g);
  return launch_status("w8a8_gemm_dma_kernel");
}

// Compute units of the current device (cached per device; concurrent first
// calls store the same value).
static int device_cus() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (!n) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Tile shape by the share of the device's tile slots, over the rounds the
// problem takes, that hold useful work (the output area M x N over all the
// slot-tiles of those rounds, so a tile's padding past M or N counts as
// waste), weighted by each shape's per-tile efficiency (measured): 256 x 256
// (the DMA-fed 4-wave kernel when K % 256 == 0, else 8 waves; 1 per CU),
// 192 (n) x 256 (m) on 8 waves (1 per CU, wave tiles 96 x 64), 128 x 128 on
// 4 waves (2 per CU). A 4096 x 9216 problem, say, is 576 tiles of
// 256 x 256 (2.25 rounds on 256 CUs) but exactly 768 of 192 x 256. The
// 128 x 128 tiles lose less to their prologue and epilogue the shorter K is:
// measured on the SD1.5 / SDXL / FLUX shapes, they match or beat the larger
// tiles at equal fill below K = 3072 when they take one round (0.9), reach
// 0.75 of them over several rounds (SDXL's 8192 x 640 -> 5120: 51.7 us
// against 48.2 us for 256 x 256 tiles) and 0.7 at K = 3072 and beyond.
// 192 (n) x 128 (m) on 4 waves (1 per CU; 0.8) serves the problems whose
// 128 x 128 tiles would put two workgroups on some CUs and one on others,
// and is a candidate only when its own tiles cover at least 3/4 of the CUs
// (with fewer, every CU runs at most one tile of either shape and the
// smaller one finishes first) and pad N by at most 2% (SDXL's N = 640 pads
// to 768: 128 x 128 tiles measured 7% faster there, 11.1 against 11.9 us at
// 8192 x 640 -> 640). Measured: FLUX's 512-row text MLP up 33.2 -> 30.5 us
// and qkv 31.6 -> 27.8 us; the choice is unchanged on the other SD1.5 /
// SDXL / FLUX shapes.
// Kernel plan for a problem: DC_GEMM_PLAN_* (the choice pick_tile launches).
static int plan_tile(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw) {
  struct Cand { int bn, bm, per_cu; float eff; };
  const int cus = device_cus();
  const bool one_round_128 = ((M + 127) / 128) * ((N + 127) / 128) <= 2 * (int64_t)cus;
  const Cand cands[4] = {{256, 256, 1, 1.0f}, {192, 256, 1, 0.95f},
                         {128, 128, 2, K >= 3072 ? 0.7f : one_round_128 ? 0.9f : 0.75f}, {192, 128, 1, 0.8f}};
  int best = 0;
  float best_score = -1.0f;
  for (int i = 0; i < 4; ++i) {
    const int64_t tn = (N + cands[i].bn - 1) / cands[i].bn, tm = (M + cands[i].bm - 1) / cands[i].bm;
    if (i == 3 && (4 * tn * tm < 3 * (int64_t)cus || 50 * (tn * 192 - N) > N)) continue;
    const int64_t slots = (int64_t)cus * cands[i].per_cu;
    const int64_t rounds = (tn * tm + slots - 1) / slots;
    const double area = (double)rounds * slots * cands[i].bn * cands[i].bm;
    const float score = (float)((double)M * (double)N / area) * cands[i].eff;
    if (score > best_score) best = i, best_score = score;
  }
  if (best == 0) {
    // 256 x 256 tiles: the DMA-fed kernel when its shape conditions hold
    if (K % (4 * DBK) == 0 && 256 * lda < (int64_t(1) << 31) && 256 * ldw < (int64_t(1) << 31))
      return DC_GEMM_PLAN_DMA_256x256;
    return DC_GEMM_PLAN_256x256;
  }
  return best == 1 ? DC_GEMM_PLAN_192x256 : best == 2 ? DC_GEMM_PLAN_128x128 : DC_GEMM_PLAN_192x128;
}

template <int OUT_DT, int BIAS_DT>
static int pick_tile(GemmArgs p, hipStream_t st) {
  switch (plan_tile(p.M, p.N, p.K, p.lda, p.ldw)) {
    case DC_GEMM_PLAN_DMA_256x256: return launch_gemm_dma<OUT_DT, BIAS_DT>(p, st);
    case DC_GEMM_PLAN_256x256: return launch_gemm<Tile<2, 4, 4, 2, 1>, OUT_DT, BIAS_DT>(p, st);
    case DC_GEMM_PLAN_192x256: return launch_gemm<Tile<2, 4, 3, 2, 1>, OUT_DT, BIAS_DT>(p, st);
    case DC_GEMM_PLAN_192x128: return launch_gemm<Tile<2, 2, 3, 2, 1>, OUT_DT, BIAS_DT>(p, st);
    default: return launch_gemm<Tile<2, 2, 2, 2, 1>, OUT_DT, BIAS_DT>(p, st);
  }
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
                          void* out, int64_t ldo, int64_t M, int64_t N, hipStream_t st, int nsplit = 1,
                          int64_t split_stride = 0) {
  const int ob = OUT_DT == DC_F32 ? 4 : 2;
  if (N % 4 == 0 && lda % 4 == 0 && ldo % 4 == 0 && split_stride % 4 == 0 && aligned16(acc) && aligned16(sw) &&
      reinterpret_cast<uintptr_t>(out) % (4 * ob) == 0) {
    const int64_t n = M * (N / 4);
    hipLaunchKernelGGL((rescale_vec_kernel<OUT_DT, BIAS_DT>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       acc, lda, sx, sw, bias, out, ldo, (int)M, (int)N, nsplit, split_stride);
    return launch_status("rescale_vec_kernel");
  }
  const int64_t n = M * ((N + 3) / 4);
  hipLaunchKernelGGL((rescale_kernel<OUT_DT, BIAS_DT>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, acc, lda,
                     sx, sw, bias, out, ldo, (int)M, (int)N, nsplit, split_stride);
  return launch_status("rescale_kernel");
}

template <int OUT_DT>
static int rescale_bias(const int32_t* acc, int64_t lda, const float* sx, const float* sw, const void* bias,
                        int bias_dtype, void* out, int64_t ldo, int64_t M, int64_t N, hipStream_t st,
                        int nsplit = 1, int64_t split_stride = 0) {
  switch (bias_dtype) {
    case DC_NONE: return launch_rescale<OUT_DT, DC_NONE>(acc, lda, sx, sw, bias, out, ldo, M, N, st, nsplit, split_stride);
    case DC_F16: return launch_rescale<OUT_DT, DC_F16>(acc, lda, sx, sw, bias, out, ldo, M, N, st, nsplit, split_stride);
    case DC_BF16: return launch_rescale<OUT_DT, DC_BF16>(acc, lda, sx, sw, bias, out, ldo, M, N, st, nsplit, split_stride);
    case DC_F32: return launch_rescale<OUT_DT, DC_F32>(acc, lda, sx, sw, bias, out, ldo, M, N, st, nsplit, split_stride);
    default: return fail(DC_EINVAL, "dc_rescale: bad bias_dtype");
  }
}

// Split-K plan for problems whose 128 x 128 tiles fill at most a quarter of
// the device's workgroup slots (2 per CU), with K >= 3072, or K >= 2048 for
// the tiniest (whatever tile
// plan_tile would pick for the unsplit call: such problems leave most CUs
// idle either way; measured, a fuller or shorter problem loses more to the
// partials' round trip and the second launch than it gains): the largest
// power of two S <= 8 with S * tiles <= slots and slices of at least 512
// bytes of k, each slice a multiple of 128. Returns 1 for no split; *kslice
// is the slice.
static int splitk_plan(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw, int* kslice) {
  *kslice = (int)K;
  (void)lda; (void)ldw;
  const int64_t tiles = ((M + 127) / 128) * ((N + 127) / 128);
  const int64_t slots = 2 * (int64_t)device_cus();
  // K >= 3072, or K >= 2048 when the tiles would fill at most 1/16 of the
  // slots (SDXL's 154-row cross-attention K/V, 10-20 tiles: 14.5 -> 9.8-10.7
  // us; at 80-96 tiles a 2048-deep split measured 30-50% slower)
  if (K < 2048 || (K < 3072 && 16 * tiles > slots)) return 1;
  if (4 * tiles > slots) return 1;
  int s = 1;
  while (s < 8 && 2 * s * tiles <= slots && K / (2 * s) >= 512) s *= 2;
  if (s == 1) return 1;
  const int64_t slice = ((K + s - 1) / s + 127) / 128 * 128;
  *kslice = (int)slice;
  return (int)((K + slice - 1) / slice);
}

}  // namespace dc

using namespace dc;

extern "C" int dc_w8a8_gemm_plan(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw) {
  clear_error();
  if (M <= 0 || N <= 0 || K <= 0 || K % 16 || lda < K || ldw < K || lda % 16 || ldw % 16) {
    set_error("dc_w8a8_gemm_plan: no kernel takes this shape");
    return -1;
  }
  return plan_tile(M, N, K, lda, ldw);
}

extern "C" size_t dc_w8a8_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 16 || lda < K || ldw < K || lda % 16 || ldw % 16) return 0;
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff) return 0;
  int kslice = 0;
  const int s = splitk_plan(M, N, K, lda, ldw, &kslice);
  return s > 1 ? (size_t)s * (size_t)M * (size_t)N * 4 : 0;
}

extern "C" int dc_w8a8_gemm(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, const float* sx,
                            const float* sw, const void* bias, int bias_dtype, void* out, int out_dtype, int64_t ldo,
                            int64_t M, int64_t N, int64_t K, void* workspace, size_t ws_bytes, void* stream) {
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
  p.vec16 = p.vec_out && (reinterpret_cast<uintptr_t>(out) % 16) == 0 && (ldo * ob) % 16 == 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (out_dtype != DC_I32 && out_dtype != DC_F16 && out_dtype != DC_BF16 && out_dtype != DC_F32)
    return fail(DC_EINVAL, "dc_w8a8_gemm: bad out_dtype");
  if (bias_dtype != DC_NONE && bias_dtype != DC_F16 && bias_dtype != DC_BF16 && bias_dtype != DC_F32)
    return fail(DC_EINVAL, "dc_w8a8_gemm: bad bias_dtype");
  // split-K into the workspace (int32 partials), then the epilogue over their sum
  int kslice = 0;
  const int ks = (out_dtype != DC_I32 && workspace) ? splitk_plan(M, N, K, lda, ldw, &kslice) : 1;
  if (ks > 1 && ws_bytes >= (size_t)ks * (size_t)M * (size_t)N * 4 && aligned16(workspace)) {
    GemmArgs q = p;
    q.sx = nullptr; q.sw = nullptr; q.bias = nullptr;
    q.out = workspace;
    q.ldo = N;
    q.vec_out = N % 4 == 0;
    q.vec16 = N % 4 == 0;
    q.ksplit = ks;
    q.kslice = kslice;
    q.split_stride = M * N;
    if (int e = launch_gemm<Tile<2, 2, 2, 2, 1>, DC_I32, DC_NONE>(q, st)) return e;
    const int32_t* acc = static_cast<const int32_t*>(workspace);
    switch (out_dtype) {
      case DC_F16: return rescale_bias<DC_F16>(acc, N, sx, sw, bias, bias_dtype, out, ldo, M, N, st, ks, M * N);
      case DC_BF16: return rescale_bias<DC_BF16>(acc, N, sx, sw, bias, bias_dtype, out, ldo, M, N, st, ks, M * N);
      default: return rescale_bias<DC_F32>(acc, N, sx, sw, bias, bias_dtype, out, ldo, M, N, st, ks, M * N);
    }
  }
  switch (out_dtype) {
    case DC_I32: return pick_tile<DC_I32, DC_NONE>(p, st);
    case DC_F16: return dispatch_bias<DC_F16>(p, bias_dtype, st);
    case DC_BF16: return dispatch_bias<DC_BF16>(p, bias_dtype, st);
    case DC_F32: return dispatch_bias<DC_F32>(p, bias_dtype, st);
    default: return fail(DC_EINVAL, "dc_w8a8_gemm: bad out_dtype");
  }
}

// ---------------------------------------------------------------- grouped launches

template <int OUT_DT, bool RES = false>
static int group_bias(GemmArgs p, const GroupArgs& g, int bias_dtype, hipStream_t st) {
  switch (bias_dtype) {
    case DC_NONE: return launch_gemm_dma_group<OUT_DT, DC_NONE, RES>(p, g, st);
    case DC_F16: return launch_gemm_dma_group<OUT_DT, DC_F16, RES>(p, g, st);
    case DC_BF16: return launch_gemm_dma_group<OUT_DT, DC_BF16, RES>(p, g, st);
    default: return launch_gemm_dma_group<OUT_DT, DC_F32, RES>(p, g, st);
  }
}

static int64_t dma_tiles(int64_t M, int64_t N) { return ((M + 255) / 256) * ((N + 255) / 256); }

extern "C" int dc_w8a8_gemm_group_plan(const int64_t* Ms, int count, int64_t N, int64_t K) {
  clear_error();
  if (!Ms || count < 1 || count > DC_GEMM_MAX_GROUP || N <= 0 || K <= 0) {
    set_error("dc_w8a8_gemm_group_plan: bad arguments");
    return -1;
  }
  int live = 0;
  int64_t total = 0, largest = 0;
  for (int i = 0; i < count; ++i) {
    if (Ms[i] < 0) {
      set_error("dc_w8a8_gemm_group_plan: negative M");
      return -1;
    }
    if (Ms[i] == 0) continue;
    ++live;
    const int64_t t = dma_tiles(Ms[i], N);
    total += t;
    largest = t > largest ? t : largest;
  }
  if (K % (4 * DBK) || live < 2) return 0;
  const int64_t cus = device_cus();
  return (total + cus - 1) / cus <= (largest + cus - 1) / cus ? 1 : 0;
}

static int group_fail(int code, const char* who, const char* msg) {
  set_error("%s: %s", who, msg);
  return code;
}

// Checks and per-problem set-up shared by the grouped entry points. gates:
// NULL, or one dc_gemm_gate per problem (the gated residual). An error
// message starts with `who`.
static int group_setup(const char* who, const dc_gemm_problem* problems, const dc_gemm_gate* gates, int count,
                       int64_t N, int64_t K, int bias_dtype, int out_dtype, GemmArgs& p, GroupArgs& g) {
  if (!problems) return group_fail(DC_EINVAL, who, "null pointer");
  if (count < 1 || count > DC_GEMM_MAX_GROUP) return group_fail(DC_EINVAL, who, "count must be 1 .. DC_GEMM_MAX_GROUP");
  if (N <= 0 || K <= 0) return group_fail(DC_EINVAL, who, "N and K must be positive");
  if (N > 0x7fffffff || K > 0x7fffffff) return group_fail(DC_EINVAL, who, "size too large");
  if (K % (4 * DBK)) return group_fail(DC_EUNSUPPORTED, who, "needs K % 256 == 0");
  if (out_dtype != DC_I32 && out_dtype != DC_F16 && out_dtype != DC_BF16 && out_dtype != DC_F32)
    return group_fail(DC_EINVAL, who, "bad out_dtype");
  if (bias_dtype != DC_NONE && bias_dtype != DC_F16 && bias_dtype != DC_BF16 && bias_dtype != DC_F32)
    return group_fail(DC_EINVAL, who, "bad bias_dtype");
  const int ob = elem_bytes(out_dtype);
  p = GemmArgs{};
  p.N = (int)N;
  p.K = (int)K;
  p.tiles_n = (int)((N + 255) / 256);
  g = GroupArgs{};
  int64_t tiles = 0;
  for (int i = 0; i < count; ++i) {
    const dc_gemm_problem& q = problems[i];
    if (q.M < 0) return group_fail(DC_EINVAL, who, "negative M");
    if (q.M == 0) continue;
    if (q.M > 0x7fffffff) return group_fail(DC_EINVAL, who, "size too large");
    if (!q.a || !q.w || !q.out) return group_fail(DC_EINVAL, who, "null pointer");
    if (q.lda < K || q.ldw < K || q.lda % 16 || q.ldw % 16 || !aligned16(q.a) || !aligned16(q.w) ||
        256 * q.lda >= (int64_t(1) << 31) || 256 * q.ldw >= (int64_t(1) << 31))
      return group_fail(DC_EUNSUPPORTED, who,
                        "needs lda, ldw >= K, multiples of 16 and below 2^23, 16-byte aligned a, w");
    if (q.ldo < N) return group_fail(DC_EINVAL, who, "ldo < N");
    if (out_dtype != DC_I32 && (!q.sx || !q.sw)) return group_fail(DC_EINVAL, who, "scales are required");
    if (bias_dtype != DC_NONE && out_dtype != DC_I32 && !q.bias)
      return group_fail(DC_EINVAL, who, "bias_dtype given without bias");
    GroupProblem& d = g.prob[g.ngroup];
    d.a = q.a; d.w = q.w; d.sx = q.sx; d.sw = q.sw; d.bias = q.bias; d.out = q.out;
    d.lda = q.lda; d.ldw = q.ldw; d.ldo = q.ldo;
    d.M = (int)q.M;
    d.tiles_m = (int)((q.M + 255) / 256);
    d.vec_out = ((reinterpret_cast<uintptr_t>(q.out) % (4 * (uintptr_t)ob)) == 0) && (q.ldo % 4 == 0) &&
                (out_dtype == DC_I32 || (reinterpret_cast<uintptr_t>(q.sw) & 15) == 0);
    d.vec16 = d.vec_out && (reinterpret_cast<uintptr_t>(q.out) % 16) == 0 && (q.ldo * ob) % 16 == 0;
    if (gates) {
      const dc_gemm_gate& r = gates[i];
      if (!r.res || !r.gate) return group_fail(DC_EINVAL, who, "null residual or gate");
      if (r.ldr < N) return group_fail(DC_EINVAL, who, "ldr < N");
      // in place, each output element must read only its own residual
      // element: other row strides would read rows other tiles overwrite
      if (r.res == q.out && r.ldr != q.ldo)
        return group_fail(DC_EINVAL, who, "a residual that is the output needs ldr == ldo");
      d.res = r.res; d.gate = r.gate; d.ldr = r.ldr;
      // the residual's loads follow the output's stores, so they need the same alignment
      d.vec_out = d.vec_out && (reinterpret_cast<uintptr_t>(r.res) % (4 * (uintptr_t)ob)) == 0 && r.ldr % 4 == 0;
      d.vec16 = d.vec16 && d.vec_out && (reinterpret_cast<uintptr_t>(r.res) % 16) == 0 && (r.ldr * ob) % 16 == 0;
    }
    g.first[g.ngroup] = (int)tiles;
    tiles += (int64_t)d.tiles_m * p.tiles_n;
    if (tiles > 0x7fffffff) return group_fail(DC_EINVAL, who, "problem too large");
    ++g.ngroup;
  }
  g.first[g.ngroup] = (int)tiles;
  return DC_OK;
}

extern "C" int dc_w8a8_gemm_grouped(const dc_gemm_problem* problems, int count, int64_t N, int64_t K, int bias_dtype,
                                    int out_dtype, void* stream) {
  clear_error();
  GemmArgs p;
  GroupArgs g;
  if (int e = group_setup("dc_w8a8_gemm_grouped", problems, nullptr, count, N, K, bias_dtype, out_dtype, p, g))
    return e;
  if (g.ngroup == 0) return DC_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (out_dtype) {
    case DC_I32: return launch_gemm_dma_group<DC_I32, DC_NONE>(p, g, st);
    case DC_F16: return group_bias<DC_F16>(p, g, bias_dtype, st);
    case DC_BF16: return group_bias<DC_BF16>(p, g, bias_dtype, st);
    default: return group_bias<DC_F32>(p, g, bias_dtype, st);
  }
}

extern "C" int dc_w8a8_gemm_grouped_gated(const dc_gemm_problem* problems, const dc_gemm_gate* gates, int count,
                                          int64_t N, int64_t K, int bias_dtype, int out_dtype, void* stream) {
  clear_error();
  const char* who = "dc_w8a8_gemm_grouped_gated";
  if (!gates) return group_fail(DC_EINVAL, who, "null pointer");
  if (out_dtype != DC_F16 && out_dtype != DC_BF16 && out_dtype != DC_F32)
    return group_fail(DC_EINVAL, who, "out_dtype must be DC_F16, DC_BF16 or DC_F32");
  GemmArgs p;
  GroupArgs g;
  if (int e = group_setup(who, problems, gates, count, N, K, bias_dtype, out_dtype, p, g)) return e;
  if (g.ngroup == 0) return DC_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (out_dtype) {
    case DC_F16: return group_bias<DC_F16, true>(p, g, bias_dtype, st);
    case DC_BF16: return group_bias<DC_BF16, true>(p, g, bias_dtype, st);
    default: return group_bias<DC_F32, true>(p, g, bias_dtype, st);
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
  if (M > 0x7fffffff || N > 0x7fffffff || M * ((N + 3) / 4) > (int64_t)0x7fffffff * 256)
    return fail(DC_EINVAL, "dc_rescale: size too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (out_dtype) {
    case DC_F16: return rescale_bias<DC_F16>(acc, lda, sx, sw, bias, bias_dtype, out, ldo, M, N, st);
    case DC_BF16: return rescale_bias<DC_BF16>(acc, lda, sx, sw, bias, bias_dtype, out, ldo, M, N, st);
    case DC_F32: return rescale_bias<DC_F32>(acc, lda, sx, sw, bias, bias_dtype, out, ldo, M, N, st);
    default: return fail(DC_EINVAL, "dc_rescale: bad out_dtype");
  }
}
