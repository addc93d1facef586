// INT8-QK / 16-bit-PV flash attention for gfx950.
//
// Replaces fwd() of the reference (src/diffucore/kernels/int8_attn_sm80.cu:460-497)
// and extends it from fp16 / head_dim 128 to fp16 or bf16 and any head dim
// D <= 128 with D % 8 == 0 (padded to Dp = 64 or 128 inside the kernels).
//
// Kernels, in launch order (all on the caller's stream):
//  1. kstats_kernel  per-window per-channel key sums in the reference's fixed
//                    float32 order (int8_attn_sm80.cu:92-135, K half only: the V
//                    bound that kernel also computes guards fp16 PV partials,
//                    which this path does not have - PV accumulates in fp32).
//  2. kquant_kernel  ksum = sequential sum over windows (:137-142); K smoothed by
//                    its mean, val = fma(-ksum, 1/L, k), quantized per 64-key
//                    block (:38-90) into the workspace.
//  3. attn_wide_kernel or attn_kernel (+ attn_merge_kernel for stream-K plans)
//                    Q quantized per token in-kernel (:341-388); S^T = K Q^T on
//                    v_mfma_i32_32x32x32_i8 (int32, exact); base-2 online softmax
//                    in float32 on the logits S * (qs*sm_scale*log2e * ks_block);
//                    P rounded to the 16-bit input type; O^T = V^T P^T on
//                    v_mfma_f32_32x32x16_{bf16,f16} with float32 accumulation.
//                    attn_wide_kernel (K / V DMA-fed into an LDS ring) runs
//                    whole 256-row query tiles at Dp = 128 when they fill a
//                    workgroup per CU, and every Dp = 64 plan (128-row tiles,
//                    stream-K pieces included); attn_kernel runs the rest
//                    (smaller Dp = 128 grids, V row strides past 2^23).
//
// attn_kernel: a workgroup owns 128 query rows of one (batch, head), 4 waves x
// 32 rows. Computing S^T and O^T (instead of S and O) makes every accumulator
// a lane holds belong to the lane's own query row (lane % 32): the row max, row
// sum and rescale are per-lane scalars and P feeds the PV MFMA from registers.
// K (int8, from the workspace) and V (16-bit, read in place from the caller's
// strided tensor) stream through two LDS stages of 64 keys; V^T operands come
// out of LDS with ds_read_tr16_b64, which transposes 4 keys x 16 channels per
// 16 lanes. The int32 score accumulators start at 0x4B400000, so each holds
// the float32 bit pattern of 12582912 + S (exact for |S| < 2^22) and the
// exponent c*S - m is one FMA (the reference's magic-number conversion,
// int8_attn_sm80.cu:33-34, 263, 275, with its integer add folded into the MFMA).
#include "common.h"

#include <algorithm>
#include <atomic>
#include <mutex>

namespace dc {

constexpr int BQ = 128;   // query rows per workgroup
constexpr int BKEY = 64;  // keys per tile / per K scale block
constexpr int WIN = 128;  // keys per column-sum window
constexpr int MAGIC_I = 0x4B400000;
constexpr float MAGIC_F = 12582912.0f;

typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s* lds_v4s_ptr;

struct AttnArgs {
  const void* q; const void* k; const void* v; void* o;
  int8_t* k8; float* ks; float* kpart; float* ksum;
  float* part;   // stream-K partial results: slots of attn_part_floats<DP>() floats
  int B, H, Lq, Lk, D, Lk64, nwin;
  // work split of the attention kernel: blocks 0 .. dp_blocks - 1 run query
  // tiles 0 .. dp_blocks - 1 whole; the sk_blocks blocks after them share the
  // (query tile, key tile) pairs of the last sk_tiles query tiles
  int dp_blocks, sk_blocks, sk_tiles;
  int wide;   // 1: attn_wide_kernel runs the dp_blocks query tiles (Wide<Dp>::BQW rows each)
  int64_t qsb, qsl, qsh, ksb, ksl, ksh, vsb, vsl, vsh, osb, osl, osh;
  float scale_log2;
};

// most stream-K pieces one query tile is split into (attn_plan keeps to it)
constexpr int ATTN_MAX_PIECES = 8;

// floats per partial-result slot: O [BQ][DP], then the row maxima and row sums
template <int DP>
constexpr int attn_part_floats() { return BQ * DP + 2 * BQ; }

// Blocks i = 0 .. n - 1 in an order that gives each XCD (the hardware deals
// blocks round-robin over 8) a contiguous range.
__device__ __forceinline__ int xcd_order(int i, int n) { return (n % 8 == 0) ? (i % 8) * (n / 8) + i / 8 : i; }

// First (query tile, key tile) unit of stream-K block w of sk_blocks, over
// units = sk_tiles * ntiles units.
__host__ __device__ __forceinline__ int64_t sk_first(int64_t w, int64_t units, int64_t sk_blocks) {
  return w * units / sk_blocks;
}

template <int DT>
__device__ __forceinline__ void unpack8(uint4 u, float (&f)[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = h16_to_f32<DT>(w[i] & 0xffffu);
    f[2 * i + 1] = h16_to_f32<DT>(w[i] >> 16);
  }
}

// Four codes rint(f[i] * inv) as bytes of one word. The product is rounded
// to float32 first; adding 1.5 * 2^23 then rounds it to an integer n, ties to
// even, exactly as rintf does (|product| < 2^22: the codes are within
// +-128), and leaves the bits 0x4B400000 + n, whose low byte is n as an int8.
// Two byte permutes and an or gather the four low bytes.
__device__ __forceinline__ uint32_t pack_codes(const float* f, float inv) {
  uint32_t b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) b[i] = __float_as_uint(materialize(f[i] * inv) + MAGIC_F);
  // v_perm_b32 selector bytes: 0..3 pick bytes of the second operand, 4..7
  // of the first, 0x0c gives 0
  return __builtin_amdgcn_perm(b[1], b[0], 0x0c0c0400u) | __builtin_amdgcn_perm(b[3], b[2], 0x04000c0cu);
}

// ---------------------------------------------------------------- 1. key sums

template <int DT>
__global__ void __launch_bounds__(256) kstats_kernel(AttnArgs p) {
  const int w = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int t = threadIdx.x, rg = t >> 4, ch = t & 15;
  float ak[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (ch * 8 < p.D) {
    // the thread's 8 keys w * WIN + rg + 16 i, loaded together (keys past Lk
    // read key Lk - 1 and are zeroed), then summed in increasing key order
    const uint16_t* kb = static_cast<const uint16_t*>(p.k) + b * p.ksb + h * p.ksh + ch * 8;
    const int r0 = w * WIN + rg;
    uint4 raw[WIN / 16];
#pragma unroll
    for (int i = 0; i < WIN / 16; ++i)
      raw[i] = *reinterpret_cast<const uint4*>(kb + (int64_t)min(r0 + 16 * i, p.Lk - 1) * p.ksl);
#pragma unroll
    for (int i = 0; i < WIN / 16; ++i) {
      const bool in = r0 + 16 * i < p.Lk;
      const uint4 u = make_uint4(in ? raw[i].x : 0u, in ? raw[i].y : 0u, in ? raw[i].z : 0u, in ? raw[i].w : 0u);
      float f[8];
      unpack8<DT>(u, f);
#pragma unroll
      for (int e = 0; e < 8; ++e) ak[e] += f[e];   // + 0 leaves a sum that started at +0 unchanged
    }
  }
  // The 16 row groups' partial sums, then each channel's 16 partials added in
  // row-group order. Row group rg keeps channels 8 ch + 0..3 at float
  // 4 ch + 0..3 and 8 ch + 4..7 at 96 + 4 ch + 0..3 of its row of RP floats:
  // the 16 lanes of one row group write 256 contiguous bytes per half. A read
  // instruction takes two rows (ds_read2_b32), and 32 lanes' channels sit on
  // 32 banks of a row; RP = 16 (mod 64) puts the next row's copies on the
  // other 32 (a 160-float pitch, 32 mod 64, put them on the same ones).
  constexpr int RP = 208;
  __shared__ __attribute__((aligned(16))) float red[16 * RP];
  if (ch * 8 < p.D) {
    *reinterpret_cast<float4*>(red + rg * RP + 4 * ch) = make_float4(ak[0], ak[1], ak[2], ak[3]);
    *reinterpret_cast<float4*>(red + rg * RP + 96 + 4 * ch) = make_float4(ak[4], ak[5], ak[6], ak[7]);
  }
  __syncthreads();
  if (t < p.D) {
    const int idx = ((t & 4) ? 96 : 0) + 4 * (t >> 3) + (t & 3);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) s += red[i * RP + idx];
    p.kpart[((int64_t)(b * p.H + h) * p.nwin + w) * p.D + t] = s;
  }
}

// ---------------------------------------------------------------- 2. K quantize

// 64-key blocks per kquant workgroup: one per wave, so a block's absmax is a
// wave reduction and the window sum is read once per KQ_BLOCKS blocks
constexpr int KQ_BLOCKS = 4;

// A workgroup takes blocks KQ_BLOCKS g .. + 3 of one (b, h), wave wv block
// KQ_BLOCKS g + wv. Lane l covers channels 16 cp .. 16 cp + 15 (cp = l % LPR)
// of key rows l / LPR + RPP j: two 16-byte loads and one 16-byte store of
// codes per row.
template <int DT, int DP>
__global__ void __launch_bounds__(256) kquant_kernel(AttnArgs p) {
  constexpr int LPR = DP / 16;          // lanes per key row
  constexpr int RPP = 64 / LPR;         // rows per pass of the wave
  constexpr int NP = BKEY / RPP;        // passes over the block
  const int g = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int bh = b * p.H + h, t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int nblk = p.Lk64 / BKEY;
  const int blk = KQ_BLOCKS * g + wv;
  // the window sums, 4 floats of padding after channel 63: the float4 reads
  // of the lanes' 16-channel slices then fall in distinct banks (channel 64 c
  // would share a bank with channel 0 unpadded)
  __shared__ __attribute__((aligned(16))) float ksum_s[128 + 4];

  // the block's key loads first (clamped in bounds: a wave past the last
  // block reads it again, rows past Lk read row Lk - 1, chunks past D the last
  // chunk inside D; none of those values is used), so they are in flight
  // while the window sums are read and added
  const int cp = lane % LPR, r0 = lane / LPR;
  const int c0 = min(2 * cp, p.D / 8 - 1), c1 = min(2 * cp + 1, p.D / 8 - 1);
  const uint16_t* kb = static_cast<const uint16_t*>(p.k) + b * p.ksb + h * p.ksh;
  const int k0 = min(blk, nblk - 1) * BKEY;
  uint4 raw[NP][2];
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int64_t row = min(k0 + r0 + RPP * j, p.Lk - 1) * p.ksl;
    raw[j][0] = *reinterpret_cast<const uint4*>(kb + row + c0 * 8);
    raw[j][1] = *reinterpret_cast<const uint4*>(kb + row + c1 * 8);
  }

  if (t < p.D) {
    // sequential sum over windows, 16 window loads in flight at a time
    const float* kp = p.kpart + (int64_t)bh * p.nwin * p.D + t;
    float s = 0.f;
    for (int w0 = 0; w0 < p.nwin; w0 += 16) {
      float part[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) part[i] = kp[(int64_t)min(w0 + i, p.nwin - 1) * p.D];
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (w0 + i < p.nwin) s += part[i];
    }
    ksum_s[t + 4 * (t >> 6)] = s;
    if (g == 0) p.ksum[(int64_t)bh * p.D + t] = s;
  }
  __syncthreads();
  if (blk >= nblk) return;

  // the lane's 16 channel sums (channels past D: 0, their values are zeroed)
  const bool in0 = 16 * cp < p.D, in1 = 16 * cp + 8 < p.D;
  float km[16];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const bool in = hh ? in1 : in0;
    const int c0 = 16 * cp + 8 * hh, c1 = c0 + 4;   // channel groups of 4, padded index below
    const float4 a = in ? *reinterpret_cast<const float4*>(ksum_s + c0 + 4 * (c0 >> 6)) : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 c = in ? *reinterpret_cast<const float4*>(ksum_s + c1 + 4 * (c1 >> 6)) : make_float4(0.f, 0.f, 0.f, 0.f);
    km[8 * hh] = a.x; km[8 * hh + 1] = a.y; km[8 * hh + 2] = a.z; km[8 * hh + 3] = a.w;
    km[8 * hh + 4] = c.x; km[8 * hh + 5] = c.y; km[8 * hh + 6] = c.z; km[8 * hh + 7] = c.w;
  }
  const float inv_l = 1.f / (float)p.Lk;
  float val[NP][16];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const bool rin = k0 + r0 + RPP * j < p.Lk;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      float f[8];
      unpack8<DT>(raw[j][hh], f);
      const bool in = rin && (hh ? in1 : in0);
#pragma unroll
      for (int i = 0; i < 8; ++i) val[j][8 * hh + i] = in ? __builtin_fmaf(-km[8 * hh + i], inv_l, f[i]) : 0.f;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(val[j][i]));
  }
  amax = wave_max(amax);
  const float inv = amax > 0.f ? 127.f / amax : 0.f;
  if (lane == 0) p.ks[(int64_t)bh * nblk + blk] = amax / 127.f;
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    int8_t* dst = p.k8 + ((int64_t)bh * p.Lk64 + k0 + r0 + RPP * j) * DP + 16 * cp;
    *reinterpret_cast<uint4*>(dst) = make_uint4(pack_codes(val[j], inv), pack_codes(val[j] + 4, inv),
                                                pack_codes(val[j] + 8, inv), pack_codes(val[j] + 12, inv));
  }
}

// ---------------------------------------------------------------- Q quantize (shared)

// Quantizes query row `row` for the S^T MFMA: lane half hf owns channels
// 32 ks + 16 hf + 0..15 (ks < Dp / 32), so the two halves of a 32-lane column
// hold the whole row. q8 = rint(q * (127 / amax)); returns qs = amax / 127.
template <int DT, int DP>
__device__ __forceinline__ float quantize_q_row(const uint16_t* qrow, bool valid, int D, int hf,
                                                v4i (&qf)[DP / 32]) {
  constexpr int ND = DP / 32;
  float f[ND][16];
  float amax = 0.f;
  uint4 raw[ND][2];
#pragma unroll
  for (int ks = 0; ks < ND; ++ks)   // all loads first; channels past D read channel 0 and are zeroed
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int c0 = 32 * ks + 16 * hf + 8 * hh;
      raw[ks][hh] = *reinterpret_cast<const uint4*>(qrow + (c0 < D ? c0 : 0));
    }
#pragma unroll
  for (int ks = 0; ks < ND; ++ks)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const bool in = valid && 32 * ks + 16 * hf + 8 * hh < D;
      const uint4 u = make_uint4(in ? raw[ks][hh].x : 0u, in ? raw[ks][hh].y : 0u, in ? raw[ks][hh].z : 0u,
                                 in ? raw[ks][hh].w : 0u);
      unpack8<DT>(u, *reinterpret_cast<float(*)[8]>(&f[ks][8 * hh]));
    }
#pragma unroll
  for (int ks = 0; ks < ND; ++ks)
#pragma unroll
    for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(f[ks][i]));
  amax = fmaxf(amax, __shfl_xor(amax, 32));
  const float inv = amax > 0.f ? 127.f / amax : 0.f;
#pragma unroll
  for (int ks = 0; ks < ND; ++ks)
#pragma unroll
    for (int i = 0; i < 4; ++i) qf[ks][i] = (int)pack_codes(&f[ks][4 * i], inv);
  return amax / 127.f;
}

// Debug / verification entry: the same per-token quantizer, codes to memory.
template <int DT, int DP>
__global__ void __launch_bounds__(64) qquant_kernel(AttnArgs p, int8_t* q8, float* qs, int Lq32) {
  const int lane = threadIdx.x, hf = lane >> 5, l32 = lane & 31;
  const int bh = blockIdx.y, b = bh / p.H, h = bh % p.H;
  const int row = blockIdx.x * 32 + l32;
  const bool valid = row < p.Lq;
  const uint16_t* qrow = static_cast<const uint16_t*>(p.q) + b * p.qsb + (int64_t)(valid ? row : 0) * p.qsl + h * p.qsh;
  v4i qf[DP / 32];
  const float s = quantize_q_row<DT, DP>(qrow, valid, p.D, hf, qf);
  int8_t* dst = q8 + ((int64_t)bh * Lq32 + row) * DP + 16 * hf;
#pragma unroll
  for (int ks = 0; ks < DP / 32; ++ks) *reinterpret_cast<v4i*>(dst + 32 * ks) = qf[ks];
  if (hf == 0) qs[(int64_t)bh * Lq32 + row] = s;
}

// ---------------------------------------------------------------- 3. attention

template <int DT>
__device__ __forceinline__ v16f mfma_pv(const v4i a, const v4i b, v16f c) {
  if constexpr (DT == DC_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0, 0);
}

template <int DT>
__device__ __forceinline__ uint32_t pack_probs16(float a, float b) {
  v2f x = {a, b};
  if constexpr (DT == DC_BF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, v2bf));
  else return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, v2h));
}

// acc + p.x + p.y of a packed pair (v_dot2c_f32_{bf16,f16} against (1, 1))
template <int DT>
__device__ __forceinline__ float sum2(uint32_t pk, float acc) {
  if constexpr (DT == DC_BF16) {
    const v2bf one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, pk), one, acc, false);
  } else {
    const v2h one = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2h, pk), one, acc, false);
  }
}

// One 64-key tile for the wave's 32 query rows: S^T = K Q^T, online softmax,
// O^T += V^T P^T. TAIL masks keys at and past Lk (last tile only).
// S^T[key][q] + magic for one 64-key tile: block kb covers keys 32 kb .. +31;
// register j of block kb holds key 32 kb + 8 (j / 4) + 4 hf + j % 4.
template <int DP>
__device__ __forceinline__ void qk_tile(const uint8_t* __restrict__ sK, int klane, const v4i (&qf)[DP / 32],
                                        v16i (&s)[2]) {
  constexpr int KP = DP + 16, ND = DP / 32;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int j = 0; j < 16; ++j) s[kb][j] = MAGIC_I;
#pragma unroll
  for (int ks = 0; ks < ND; ++ks)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const v4i a = *reinterpret_cast<const v4i*>(sK + klane + (32 * kb) * KP + 32 * ks);
      s[kb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, qf[ks], s[kb], 0, 0, 0);
    }
}

__device__ __forceinline__ int max3i(int a, int b, int c) { return max(max(a, b), c); }

// Online softmax of one tile: P = 2^(bits(S) * c - bias) as 16-bit pairs (bias
// = MAGIC_F c + m: the scores carry the bits of 12582912 + S), and its sum
// added to lsum (the packed values, v_dot2c against (1, 1)). key0 is the key
// of register 0 of block 0 for this lane (tile start + 4 hf); TAIL zeroes keys
// >= Lk.
template <int DT, bool TAIL>
__device__ __forceinline__ void softmax_exp(const v16i (&s)[2], int key0, int Lk, float c, float bias, float& lsum,
                                            uint32_t (&pk)[2][8]) {
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int j = 0; j < 16; j += 2) {
      float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(__int_as_float(s[kb][j]), c, -bias));
      float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(__int_as_float(s[kb][j + 1]), c, -bias));
      if constexpr (TAIL) {
        if (key0 + 32 * kb + 8 * (j >> 2) + (j & 3) >= Lk) p0 = 0.f;
        if (key0 + 32 * kb + 8 * (j >> 2) + (j & 3) + 1 >= Lk) p1 = 0.f;
      }
      pk[kb][j >> 1] = pack_probs16<DT>(p0, p1);
      lsum = sum2<DT>(pk[kb][j >> 1], lsum);
    }
}

// O^T[d][q] += V^T[d][keys] P^T[keys][q], 16 keys per MFMA.
template <int DT, int DP>
__device__ __forceinline__ void pv_tile(const uint32_t (&pk)[2][8], const uint8_t* __restrict__ sV, int vlane,
                                        v16f (&o)[DP / 32]) {
  constexpr int VP = 2 * DP + 64, ND = DP / 32;
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const int kb = kk >> 1, j0 = 4 * (kk & 1);
    const v4i pf = {(int)pk[kb][j0], (int)pk[kb][j0 + 1], (int)pk[kb][j0 + 2], (int)pk[kb][j0 + 3]};
#pragma unroll
    for (int i = 0; i < ND; ++i) {
      // keys 16 kk + 4 hf + li / 4 (and + 8), channels 32 i + 16 g16 + 4 (li % 4) .. + 3
      const uint8_t* a = sV + vlane + (16 * kk) * VP + (32 * i) * 2;
      const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_ptr)(const_cast<uint8_t*>(a)));
      const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_ptr)(const_cast<uint8_t*>(a + 8 * VP)));
      const v4i av = {(int)((uint32_t)(uint16_t)lo[0] | ((uint32_t)(uint16_t)lo[1] << 16)),
                      (int)((uint32_t)(uint16_t)lo[2] | ((uint32_t)(uint16_t)lo[3] << 16)),
                      (int)((uint32_t)(uint16_t)hi[0] | ((uint32_t)(uint16_t)hi[1] << 16)),
                      (int)((uint32_t)(uint16_t)hi[2] | ((uint32_t)(uint16_t)hi[3] << 16))};
      o[i] = mfma_pv<DT>(av, pf, o[i]);
    }
  }
}

// Largest probability a tile may hold before the running maximum moves:
// P = 2^(logit - m) <= 2^12 keeps float16 P (max 65504) and float32 O and row
// sums in range. O / sum(P) does not depend on m.
constexpr float P_LIMIT = 4096.f;

// Exact maximum logit of the lane's query row over the tile. The scores carry
// the bits of 12582912 + S, positive floats, so integer order is float order:
// four independent max3 chains, then the lane halves (same query row, the
// other keys) exchanged with v_permlane32_swap. TAIL excludes keys >= Lk
// (their scores are overwritten).
template <bool TAIL>
__device__ __forceinline__ float tile_max(v16i (&s)[2], int key0, int Lk, float c) {
  if constexpr (TAIL) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (key0 + 32 * kb + 8 * (j >> 2) + (j & 3) >= Lk) s[kb][j] = INT_MIN;
  }
  int mq[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int kb = q >> 1, j0 = 8 * (q & 1);
    mq[q] = max3i(s[kb][j0], s[kb][j0 + 1], s[kb][j0 + 2]);
    mq[q] = max3i(mq[q], s[kb][j0 + 3], s[kb][j0 + 4]);
    mq[q] = max3i(mq[q], s[kb][j0 + 5], s[kb][j0 + 6]);
    mq[q] = max(mq[q], s[kb][j0 + 7]);
  }
  int mx = max(max(mq[0], mq[1]), max(mq[2], mq[3]));
  const auto halves = __builtin_amdgcn_permlane32_swap(mx, mx, false, false);
  mx = max((int)halves[0], (int)halves[1]);
  return (__int_as_float(mx) - MAGIC_F) * c;
}

// Lazy row maximum. The tile's P was taken against the running maximum m
// (bias = MAGIC_F c + m) and `ts` holds the lane's sum of it. When some lane's
// sum exceeds P_LIMIT (so a probability may exceed it), or at the first tile
// (m = -inf gives infinities), m moves to the exact maximum, the row sum and
// O are rescaled and P is recomputed. Then ts joins the row sum.
template <int DT, int DP, bool TAIL>
__device__ __forceinline__ void lazy_fixup(v16i (&s)[2], int key0, int Lk, float c, float& m, float& lsum, float ts,
                                           v16f (&o)[DP / 32], uint32_t (&pk)[2][8]) {
  if (__any(!(ts <= P_LIMIT))) {
    const float mnew = fmaxf(m, tile_max<TAIL>(s, key0, Lk, c));
    const float alpha = __builtin_amdgcn_exp2f(m - mnew);
    m = mnew;
    lsum *= alpha;
#pragma unroll
    for (int i = 0; i < DP / 32; ++i)
#pragma unroll
      for (int j = 0; j < 16; ++j) o[i][j] *= alpha;
    ts = 0.f;
    softmax_exp<DT, TAIL>(s, key0, Lk, c, __builtin_fmaf(MAGIC_F, c, m), ts, pk);
  }
  lsum += ts;
}

// One tile's softmax and PV without a following tile to overlap.
template <int DT, int DP, bool TAIL>
__device__ __forceinline__ void softmax_pv(v16i (&s)[2], const uint8_t* __restrict__ sV, int vlane, int key0, int Lk,
                                           float ksc, float cq, float& m, float& lsum, v16f (&o)[DP / 32]) {
  const float c = cq * ksc;
  uint32_t pk[2][8];
  float ts = 0.f;
  softmax_exp<DT, TAIL>(s, key0, Lk, c, __builtin_fmaf(MAGIC_F, c, m), ts, pk);
  lazy_fixup<DT, DP, TAIL>(s, key0, Lk, c, m, lsum, ts, o, pk);
  pv_tile<DT, DP>(pk, sV, vlane, o);
}

// Shared memory of one attention workgroup: two K stages, then two V stages.
template <int DP>
constexpr int attn_smem_bytes() { return 2 * BKEY * (DP + 16) + 2 * BKEY * (2 * DP + 64); }

// One piece of attention work: query tile `qlog` (b, h, tile in that order)
// over key tiles tb .. te - 1. slot < 0: the piece is the whole key range and
// the output is stored; otherwise the unnormalized O, the running row maxima
// and the row sums go to partial-result slot `slot`.
template <int DT, int DP, bool PIECE>
__device__ __forceinline__ void attn_piece(const AttnArgs& p, uint8_t* smem, int qlog, int tb_, int te_, int slot_) {
  // LDS rows are padded so the rows an operand read touches fall on distinct
  // banks: K rows (int8, Dp bytes) by 16 bytes - 8 consecutive rows of a
  // 16-byte MFMA read land on 8 different 16-byte bank groups; V rows (16-bit,
  // 2 Dp bytes) by 64 bytes - a transposed read covers 64 bytes of each of 4
  // rows (two 16-lane groups side by side), and a pitch of 64 modulo the
  // 256-byte bank width puts those 4 spans on disjoint banks. Every operand
  // address is then a per-lane base plus a constant.
  constexpr int KP = DP + 16;            // K row pitch (bytes)
  constexpr int VP = 2 * DP + 64;        // V row pitch (bytes)
  constexpr int KB = BKEY * KP;          // K tile bytes
  constexpr int VB = BKEY * VP;          // V tile bytes
  constexpr int KCPR = DP / 16;          // 16-byte chunks per K row
  constexpr int VCPR = DP / 8;           // 16-byte chunks per V row
  constexpr int NKL = BKEY * KCPR / 256, NVL = BKEY * VCPR / 256;
  constexpr int ND = DP / 32;            // 32-row blocks of d
  static_assert(attn_smem_bytes<DP>() == 2 * KB + 2 * VB, "LDS layout");
#define SK_STAGE(st_) (smem + (st_) * KB)
#define SV_STAGE(st_) (smem + 2 * KB + (st_) * VB)

  const int t = threadIdx.x, lane = t & 63, wv = t >> 6, hf = lane >> 5, l32 = lane & 31;
  const int nqt = (p.Lq + BQ - 1) / BQ;
  const int ntiles = p.Lk64 / BKEY;
  const bool ragged = p.Lk % BKEY != 0;      // the last tile has keys past Lk
  // a whole query tile (PIECE = false) takes its key range as compile-time facts
  const int tb = PIECE ? tb_ : 0, te = PIECE ? te_ : ntiles, slot = PIECE ? slot_ : -1;
  const int qt = qlog % nqt, bh = qlog / nqt;
  const int b = bh / p.H, h = bh % p.H;
  const int qrow = qt * BQ + wv * 32 + l32;   // this lane's query row

  const int8_t* kbase = p.k8 + (int64_t)bh * p.Lk64 * DP;
  const uint16_t* vbase = static_cast<const uint16_t*>(p.v) + b * p.vsb + h * p.vsh;
  const float* ksp = p.ks + (int64_t)bh * (p.Lk64 / BKEY);

  // Register-staged tile loads: thread t moves 16-byte chunks t + 256 u. The
  // per-lane offsets inside a tile are fixed, so a full tile's loads are a
  // uniform tile base plus constants. V channels past D are clamped to the
  // last chunk; in a ragged last tile, keys past Lk are clamped to key Lk - 1
  // (those keys get P = 0 and those channels are never stored).
  // chunk u of thread t sits 256 / CPR rows below chunk 0, at the same column
  static_assert(256 % KCPR == 0 && 256 % VCPR == 0, "chunks must tile 256 threads");
  constexpr int KRU = 256 / KCPR, VRU = 256 / VCPR;   // rows between a thread's chunks
  const int krow = t / KCPR, kcol = t % KCPR, vrow = t / VCPR, vcol = t % VCPR;
  const int koff = krow * DP + kcol * 16, kls = krow * KP + kcol * 16, vls = vrow * VP + vcol * 16;
  const int64_t voff = (int64_t)vrow * p.vsl + min(vcol, p.D / 8 - 1) * 8;
  typedef uint32_t KVec __attribute__((ext_vector_type(NKL * 4)));
  typedef uint32_t VVec __attribute__((ext_vector_type(NVL * 4)));
  KVec kst;
  VVec vst;
#define LOAD_TILE(tile_)                                                                                 \
  {                                                                                                      \
    const int kt_ = (tile_);                                                                             \
    const int8_t* kt_base = kbase + (int64_t)kt_ * BKEY * DP + koff;                                     \
    static_for<NKL>([&](auto u_) {                                                                       \
      constexpr int u = decltype(u_)::value;                                                             \
      const uint4 x_ = *reinterpret_cast<const uint4*>(kt_base + u * KRU * DP);                          \
      kst[4 * u] = x_.x; kst[4 * u + 1] = x_.y; kst[4 * u + 2] = x_.z; kst[4 * u + 3] = x_.w;            \
    });                                                                                                  \
    if (ragged && kt_ == ntiles - 1) {                                                                   \
      static_for<NVL>([&](auto u_) {                                                                     \
        constexpr int u = decltype(u_)::value;                                                           \
        const int key = min(kt_ * BKEY + vrow + u * VRU, p.Lk - 1);                                      \
        const uint4 x_ = *reinterpret_cast<const uint4*>(vbase + (int64_t)key * p.vsl +                  \
                                                         min(vcol, p.D / 8 - 1) * 8);                    \
        vst[4 * u] = x_.x; vst[4 * u + 1] = x_.y; vst[4 * u + 2] = x_.z; vst[4 * u + 3] = x_.w;          \
      });                                                                                                \
    } else {                                                                                             \
      const uint16_t* vt_base = vbase + (int64_t)kt_ * BKEY * p.vsl + voff;                              \
      static_for<NVL>([&](auto u_) {                                                                     \
        constexpr int u = decltype(u_)::value;                                                           \
        const uint4 x_ = *reinterpret_cast<const uint4*>(vt_base + (int64_t)(u * VRU) * p.vsl);          \
        vst[4 * u] = x_.x; vst[4 * u + 1] = x_.y; vst[4 * u + 2] = x_.z; vst[4 * u + 3] = x_.w;          \
      });                                                                                                \
    }                                                                                                    \
  }
#define STORE_K(stage_)                                                                                  \
  static_for<NKL>([&](auto u_) {                                                                         \
    constexpr int u = decltype(u_)::value;                                                               \
    *reinterpret_cast<uint4*>(SK_STAGE(stage_) + kls + u * KRU * KP) =                                   \
        make_uint4(kst[4 * u], kst[4 * u + 1], kst[4 * u + 2], kst[4 * u + 3]);                          \
  });
#define STORE_V(stage_)                                                                                  \
  static_for<NVL>([&](auto u_) {                                                                         \
    constexpr int u = decltype(u_)::value;                                                               \
    *reinterpret_cast<uint4*>(SV_STAGE(stage_) + vls + u * VRU * VP) =                                   \
        make_uint4(vst[4 * u], vst[4 * u + 1], vst[4 * u + 2], vst[4 * u + 3]);                          \
  });

  float m = -INFINITY, lsum = 0.f;
  v16f o[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i) o[i] = v16f{0.f};
  // ds_read_tr16_b64 addressing: 16-lane group g16 of the lane's half reads keys
  // k0 + (li / 4), channels d0 + 4 (li % 4) .. + 3 of a 16-channel segment.
  const int li = lane & 15, g16 = (lane >> 4) & 1;
  const int vlane = (4 * hf + (li >> 2)) * VP + (16 * g16 + 4 * (li & 3)) * 2;
  const int klane = l32 * KP + 16 * hf;

  // Software pipeline. Iteration `tile` issues the QK^T MFMAs of tile + 1
  // (K stage (tile + 1) & 1) ahead of the softmax of `tile`, whose VALU work
  // runs in their shadow, then PV of `tile` (V stage tile & 1). K of tile + 2
  // goes into K stage tile & 1 before the barrier (its last reader, QK of
  // `tile`, ran one iteration earlier), V of tile + 2 into V stage tile & 1
  // after it (its last reader is this iteration's PV); the registers are then
  // refilled with tile + 3.
  v16i sa[2], sb[2];
  LOAD_TILE(tb);
  // Q^T operand (B of S^T = K Q^T), quantized per token; its loads go out
  // while the first tile's are in flight
  v4i qf[ND];
  float cq;
  {
    const bool valid = qrow < p.Lq;
    const uint16_t* src = static_cast<const uint16_t*>(p.q) + b * p.qsb + (int64_t)(valid ? qrow : 0) * p.qsl + h * p.qsh;
    cq = quantize_q_row<DT, DP>(src, valid, p.D, hf, qf) * p.scale_log2;
  }
  STORE_K(0);
  STORE_V(0);
  if (te - tb > 1) {
    LOAD_TILE(tb + 1);
    STORE_K(1);
    STORE_V(1);
  }
  if (te - tb > 2) LOAD_TILE(tb + 2);
  __syncthreads();
  qk_tile<DP>(SK_STAGE(0), klane, qf, sa);

  // the next tile's 8 QK^T MFMAs, each followed by 12 of the 96 VALU
  // instructions of this tile's exponentials (fma, exp, pack, row sum)
#define ATTN_STEP(tile_, cur_, next_)                                                                    \
  {                                                                                                      \
    const int tl_ = (tile_);                                                                             \
    const int st_ = (tl_ - tb) & 1;                                                                      \
    const int key0_ = tl_ * BKEY + 4 * hf;                                                               \
    const float c_ = cq * ksp[tl_];                                                                      \
    uint32_t pk_[2][8];                                                                                  \
    float ts_ = 0.f;                                                                                     \
    qk_tile<DP>(SK_STAGE(st_ ^ 1), klane, qf, next_);                                                    \
    softmax_exp<DT, false>(cur_, key0_, p.Lk, c_, __builtin_fmaf(MAGIC_F, c_, m), ts_, pk_);             \
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * ND, 0);                                              \
    _Pragma("unroll") for (int z_ = 0; z_ < 2 * ND; ++z_) {                                              \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                                 \
      __builtin_amdgcn_sched_group_barrier(0x402, 96 / (2 * ND), 0);                                     \
    }                                                                                                    \
    __builtin_amdgcn_sched_barrier(0);                                                                   \
    lazy_fixup<DT, DP, false>(cur_, key0_, p.Lk, c_, m, lsum, ts_, o, pk_);                              \
    __builtin_amdgcn_sched_barrier(0);                                                                   \
    pv_tile<DT, DP>(pk_, SV_STAGE(st_), vlane, o);                                                       \
    __builtin_amdgcn_sched_barrier(0);                                                                   \
    if (tl_ + 2 < te) STORE_K(st_);                                                                      \
    __syncthreads();                                                                                     \
    if (tl_ + 2 < te) STORE_V(st_);                                                                      \
    if (tl_ + 3 < te) LOAD_TILE(tl_ + 3);                                                                \
    __builtin_amdgcn_sched_barrier(0);                                                                   \
  }
  // tiles tb .. te - 2, two per trip so the score buffers swap roles
  int tile = tb;
  for (; tile + 2 <= te - 1; tile += 2) {
    ATTN_STEP(tile, sa, sb);
    ATTN_STEP(tile + 1, sb, sa);
  }
  if (tile < te - 1) {
    ATTN_STEP(tile, sa, sb);
    ++tile;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) sa[kb] = sb[kb];
  }
#undef ATTN_STEP
#undef LOAD_TILE
#undef STORE_K
#undef STORE_V
  // last tile of the piece (its scores are in sa); only the last key tile has keys past Lk
  if (ragged && te == ntiles)
    softmax_pv<DT, DP, true>(sa, SV_STAGE((tile - tb) & 1), vlane, tile * BKEY + 4 * hf, p.Lk, ksp[tile], cq, m,
                             lsum, o);
  else
    softmax_pv<DT, DP, false>(sa, SV_STAGE((tile - tb) & 1), vlane, tile * BKEY + 4 * hf, p.Lk, ksp[tile], cq, m,
                              lsum, o);

  // each lane half summed its own keys
  lsum += __shfl_xor(lsum, 32);
  if (slot < 0) {
    if (qrow < p.Lq) {
      const float inv = 1.f / lsum;
      uint16_t* dst = static_cast<uint16_t*>(p.o) + b * p.osb + (int64_t)qrow * p.osl + h * p.osh;
#pragma unroll
      for (int i = 0; i < ND; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = 32 * i + 8 * g + 4 * hf;
          if (d >= p.D) continue;
          const uint32_t lo = f32_to_h16<DT>(o[i][4 * g] * inv) | (f32_to_h16<DT>(o[i][4 * g + 1] * inv) << 16);
          const uint32_t hi = f32_to_h16<DT>(o[i][4 * g + 2] * inv) | (f32_to_h16<DT>(o[i][4 * g + 3] * inv) << 16);
          *reinterpret_cast<uint2*>(dst + d) = make_uint2(lo, hi);
        }
    }
  } else {
    // unnormalized O (P = 2^(logit - m)), the running maximum m and the row sum
    float* part = p.part + (int64_t)slot * attn_part_floats<DP>();
    const int r = wv * 32 + l32;
#pragma unroll
    for (int i = 0; i < ND; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<float4*>(part + r * DP + 32 * i + 8 * g + 4 * hf) =
            make_float4(o[i][4 * g], o[i][4 * g + 1], o[i][4 * g + 2], o[i][4 * g + 3]);
    if (hf == 0) {
      part[BQ * DP + r] = m;
      part[BQ * DP + BQ + r] = lsum;
    }
  }
#undef SK_STAGE
#undef SV_STAGE
}

// Stream-K blocks w0 .. w1 hold query tile qi's pieces (block w holding unit
// x: the largest w with sk_first(w) <= x); the tile is block w's first piece
// when its range starts inside the tile, else its second.
__device__ __forceinline__ void sk_tile_blocks(const AttnArgs& p, int qi, int ntiles, int& w0, int& w1) {
  const int64_t units = (int64_t)p.sk_tiles * ntiles, S = p.sk_blocks;
  const int64_t x0 = (int64_t)qi * ntiles, x1 = x0 + ntiles - 1;
  w0 = (int)(((x0 + 1) * S - 1) / units);
  w1 = (int)(((x1 + 1) * S - 1) / units);
}

// LDS of the merge: factors [ATTN_MAX_PIECES][BQ], 1 / l [BQ] (floats), then
// the pieces' partial slots [ATTN_MAX_PIECES] (ints).
constexpr int attn_merge_lds_bytes() { return (ATTN_MAX_PIECES * BQ + BQ + ATTN_MAX_PIECES) * 4; }

// Combines the stream-K pieces of stream-K query tile qi (query tile
// dp_blocks + qi): with M = max m_i over its pieces, O = sum O_i 2^(m_i - M),
// l = sum l_i 2^(m_i - M), out = O / l (pieces in key order). One thread per
// row puts the factors 2^(m_i - M) and 1 / l in LDS (`lds`, at least
// attn_merge_lds_bytes()); then DP / 4 consecutive threads take a row's
// 16-byte groups of O, all of a thread's groups loaded together.
template <int DT, int DP>
__device__ __forceinline__ void attn_merge_tile(const AttnArgs& p, int qi, uint8_t* lds) {
  constexpr int PF = attn_part_floats<DP>(), LPR = DP / 4, PER_T = BQ * LPR / 256;
  const int ntiles = p.Lk64 / BKEY, nqt = (p.Lq + BQ - 1) / BQ;
  const int qlog = p.dp_blocks + qi, t = threadIdx.x;
  const int qt = qlog % nqt, bh = qlog / nqt, b = bh / p.H, h = bh % p.H;
  const int64_t units = (int64_t)p.sk_tiles * ntiles, S = p.sk_blocks;
  int w0, w1;
  sk_tile_blocks(p, qi, ntiles, w0, w1);
  const int np = min(w1 - w0 + 1, ATTN_MAX_PIECES);   // the planner keeps it within the bound
  float* fac = reinterpret_cast<float*>(lds);          // [ATTN_MAX_PIECES][BQ]
  float* inv_l = fac + ATTN_MAX_PIECES * BQ;           // [BQ]
  int* slot_of = reinterpret_cast<int*>(inv_l + BQ);   // [ATTN_MAX_PIECES]
  if (t < np) {
    const int w = w0 + t;
    slot_of[t] = 2 * w + (sk_first(w, units, S) / ntiles == qi ? 0 : 1);
  }
  __syncthreads();
  if (t < BQ) {
    float mi[ATTN_MAX_PIECES];
    float M = -INFINITY;
    for (int i = 0; i < np; ++i) {
      mi[i] = p.part[(int64_t)slot_of[i] * PF + BQ * DP + t];
      M = fmaxf(M, mi[i]);
    }
    float l = 0.f;
    for (int i = 0; i < np; ++i) {
      const float f = __builtin_amdgcn_exp2f(mi[i] - M);
      fac[i * BQ + t] = f;
      l += p.part[(int64_t)slot_of[i] * PF + BQ * DP + BQ + t] * f;
    }
    inv_l[t] = 1.f / l;
  }
  __syncthreads();
  uint16_t* dst0 = static_cast<uint16_t*>(p.o) + b * p.osb + h * p.osh;
  constexpr int KG = 4;   // groups per pass (register budget)
  for (int k0 = 0; k0 < PER_T; k0 += KG) {
    float4 acc[KG];
#pragma unroll
    for (int k = 0; k < KG; ++k) acc[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int i = 0; i < np; ++i) {
      const float* pc = p.part + (int64_t)slot_of[i] * PF;
#pragma unroll
      for (int k = 0; k < KG; ++k) {
        const int idx = (k0 + k) * 256 + t, r = idx / LPR, c = idx % LPR;
        const float4 v = *reinterpret_cast<const float4*>(pc + r * DP + 4 * c);
        const float f = fac[i * BQ + r];
        acc[k].x += v.x * f;
        acc[k].y += v.y * f;
        acc[k].z += v.z * f;
        acc[k].w += v.w * f;
      }
    }
#pragma unroll
    for (int k = 0; k < KG; ++k) {
      const int idx = (k0 + k) * 256 + t, r = idx / LPR, c = idx % LPR;
      const int qrow = qt * BQ + r;
      if (qrow >= p.Lq || 4 * c >= p.D) continue;
      const float inv = inv_l[r];
      const uint32_t lo = f32_to_h16<DT>(acc[k].x * inv) | (f32_to_h16<DT>(acc[k].y * inv) << 16);
      const uint32_t hi = f32_to_h16<DT>(acc[k].z * inv) | (f32_to_h16<DT>(acc[k].w * inv) << 16);
      *reinterpret_cast<uint2*>(dst0 + (int64_t)qrow * p.osl + 4 * c) = make_uint2(lo, hi);
    }
  }
}

// Blocks 0 .. dp_blocks - 1 run whole query tiles (in XCD order). The
// sk_blocks blocks after them run the stream-K share of the last sk_tiles
// query tiles: block w takes units sk_first(w) .. sk_first(w + 1) - 1 of their
// (query tile, key tile) units - the end of one query tile and the start of
// the next at most - into partial slots 2 w and 2 w + 1, which
// attn_merge_kernel combines afterwards (a separate launch: the partials of
// one tile come from blocks on different XCDs, whose L2s are not coherent
// within a launch without writing them back). Both kinds share one launch,
// so stream-K blocks start on CUs as soon as whole-tile blocks leave them.
template <int DT, int DP>
__global__ void __launch_bounds__(256, 2) attn_kernel(AttnArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[attn_smem_bytes<DP>()];
  if ((int)blockIdx.x < p.dp_blocks) {
    attn_piece<DT, DP, false>(p, smem, xcd_order(blockIdx.x, p.dp_blocks), 0, 0, -1);
    return;
  }
  const int ntiles = p.Lk64 / BKEY;
  const int blk = xcd_order(blockIdx.x - p.dp_blocks, p.sk_blocks);
  const int64_t units = (int64_t)p.sk_tiles * ntiles;
  const int64_t u_end = sk_first(blk + 1, units, p.sk_blocks);
  int64_t u = sk_first(blk, units, p.sk_blocks);
  for (int piece = 0; u < u_end; ++piece) {
    const int qi = (int)(u / ntiles), tb = (int)(u % ntiles);
    const int te = (int)min((int64_t)ntiles, tb + (u_end - u));
    if (piece) __syncthreads();   // the previous piece's last reads of the LDS stages are done
    attn_piece<DT, DP, true>(p, smem, p.dp_blocks + qi, tb, te, 2 * blk + piece);
    u += te - tb;
  }
}

// Combines the pieces of stream-K query tile blockIdx.x (attn_merge_tile).
template <int DT, int DP>
__global__ void __launch_bounds__(256) attn_merge_kernel(AttnArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[attn_merge_lds_bytes()];
  attn_merge_tile<DT, DP>(p, blockIdx.x, lds);
}


// ---------------------------------------------------------------- 3b. DMA-fed attention (attn_wide_kernel)
//
// attn_wide_kernel<DT, DP>: key ranges up to WIDE_MAX_TILES tiles.
//   Dp = 128 (head dims 65 .. 128): a workgroup owns 256 query rows of one
//     (b, h), 8 waves of 32 rows, two per SIMD, one workgroup per CU.
//   Dp = 64 (head dims <= 64): 128 query rows, 4 waves, two workgroups per CU.
// Either way the waves of a workgroup are fed by one stream of K / V tiles.
// K (int8, from the workspace) and V (16-bit, read in place) go from global
// memory straight into LDS (global_load_lds: no staging registers, no LDS
// store instructions) through a ring of ATTN_WIDE_STAGES stages of one 64-key
// tile each, loaded 3 tiles ahead: per tile and wave one DMA instruction of
// K and two of V (a 64-key tile is Dp K bytes and 2 Dp V bytes per key, and
// there are Dp / 16 waves of 64 lanes x 16 bytes). Instead of padded rows,
// XOR swizzles keep the operand reads conflict-free (0 bank conflicts
// counted at Dp = 128):
//   K row r (Dp bytes, Dp / 16 chunks of 16 B): chunk c stored at chunk
//     c ^ ((r / (256 / Dp)) % (Dp / 16)), so the rows one ds_read_b128 serves
//     per cycle cover all banks;
//   V row r (2 Dp bytes, Dp / 32 segments of 64 B): segment g stored at
//     segment g ^ ((r / (128 / Dp)) % (Dp / 32)), so the 4 rows a 16-lane
//     ds_read_b64_tr_b16 group reads lie in 4 different 64-byte bank ranges.
// The K block scales are staged in LDS once, so no global load sits in the
// loop (a uniform load there would be ordered behind the tile loads and wait
// for them). Same arithmetic as attn_kernel; the iteration is described at
// `step` below.
//
// Measured on MI355X (FLUX shape): the kernel is bound by its instruction
// stream, not by memory or synchronization. With the loads and barriers
// removed it runs within 12% of its full time, and MFMA (31% busy) and VALU
// (34% busy) work barely overlap on a SIMD: a microbenchmark of one tile's
// mix (24 MFMAs, ~100 softmax VALU instructions) runs at about the sum of
// the two alone however it is arranged.
template <int DP>
struct Wide {
  static constexpr int NW = DP / 16;                  // waves per workgroup
  static constexpr int NT = 64 * NW;                  // threads
  static constexpr int BQW = 32 * NW;                 // query rows per workgroup
  static constexpr int ND = DP / 32;                  // 32-channel blocks of d
  static constexpr int WK = BKEY * DP;                // int8 K tile bytes
  static constexpr int WV = BKEY * 2 * DP;            // 16-bit V tile bytes
  static constexpr int WSTAGE = WK + WV;              // 24 KB / 12 KB
  static constexpr int KC = DP / 16;                  // 16-byte chunks per K row
  static constexpr int KSH = DP == 128 ? 1 : 2;       // log2(K rows per 256 bytes)
  static constexpr int VR = 2 * DP;                   // V row bytes
  static constexpr int VS = DP / 32;                  // 64-byte segments per V row
  static constexpr int VSH = DP == 128 ? 0 : 1;       // log2(V rows per 256 bytes)
  static constexpr int KRW = 1024 / DP;               // K rows per wave DMA
  static constexpr int VRW = 512 / DP;                // V rows per wave DMA
  static constexpr int BLOCKS = DP == 128 ? 1 : 2;    // workgroups per CU
  static_assert(DP == 64 || DP == 128, "Dp is 64 or 128");
  static_assert(NW * KRW == BKEY && 2 * NW * VRW == BKEY, "one K and two V DMAs per wave cover a tile");
};
constexpr int ATTN_WIDE_STAGES = 4;
constexpr int WIDE_LOADS = 3;                       // DMA instructions per wave per tile: 1 K + 2 V
constexpr int WIDE_MAX_TILES = 2048;                // K block scales staged in LDS: Lk <= 131072
// V row strides (elements) below which a tile's 64 V rows span under 2^31
// bytes, so attn_wide_kernel's 32-bit DMA offsets hold them
constexpr int64_t WIDE_MAX_VSL = (int64_t)1 << 23;

// vmcnt(n) with the other counters unconstrained (gfx9 encoding: vmcnt bits
// 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
#define DC_ATTN_WAIT_VMCNT(n_) __builtin_amdgcn_s_waitcnt(((n_) & 15) | (((n_) >> 4) << 14) | (7 << 4) | (15 << 8))

typedef __attribute__((address_space(3))) void* lds_void_ptr_t;

// One DMA of 16 bytes per lane from global memory into LDS
// (global_load_lds_dwordx4 from the wave-uniform address `base` plus the
// lane's byte offset `off`; lane i's bytes land at m0 + 16 i, `lds` being the
// wave's LDS destination, a byte address in the LDS address space). Inline
// asm, so the compiler's wait-count pass does not see an LDS store: it cannot
// tell the ring stages apart and otherwise waits for every DMA in flight
// (vmcnt(0)) before some of the next tile's LDS reads, which measured 3% of
// the kernel's time at the FLUX shape. The kernel orders each stage's writes
// and reads itself, by vmcnt waits and barriers.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base),
               "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)reinterpret_cast<uintptr_t>((lds_void_ptr_t)(const_cast<void*>(p)));
}

// The 2 Dp / 32 K operands (k-step ks, key block kb) of one 64-key tile from a
// swizzled K stage; kfo[ks] is the lane's byte offset of its 16-byte chunk for
// k-step ks (row l32).
template <int DP>
__device__ __forceinline__ void k_operands(const uint8_t* __restrict__ sK, const int (&kfo)[DP / 32],
                                           v4i (&ka)[DP / 16]) {
#pragma unroll
  for (int ks = 0; ks < DP / 32; ++ks)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) ka[2 * ks + kb] = *reinterpret_cast<const v4i*>(sK + kfo[ks] + (32 * kb) * DP);
}

// S^T + magic from the K operands (`magic` holds MAGIC_I in every register: the
// first k-step accumulates onto it, so the scores need no initialization).
template <int DP>
__device__ __forceinline__ void qk_mfma(const v4i (&ka)[DP / 16], const v4i (&qf)[DP / 32], const v16i& magic,
                                        v16i (&s)[2]) {
#pragma unroll
  for (int ks = 0; ks < DP / 32; ++ks)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
      s[kb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ka[2 * ks + kb], qf[ks], ks == 0 ? magic : s[kb], 0, 0, 0);
}

// V^T operand f (16-key step kk = f / ND, channel block i = f % ND) from a
// swizzled V stage by two ds_read_tr16_b64; vfo[i] is the lane's byte offset
// for channel block i (keys 4 hf + li / 4, + 8 for the second read).
template <int DP>
__device__ __forceinline__ v4i v_operand(const uint8_t* __restrict__ sV, const int (&vfo)[DP / 32], int f) {
  constexpr int ND = DP / 32, VR = 2 * DP;
  const uint8_t* a = sV + vfo[f % ND] + (16 * (f / ND)) * VR;
  const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_ptr)(const_cast<uint8_t*>(a)));
  const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_ptr)(const_cast<uint8_t*>(a + 8 * VR)));
  return v4i{(int)((uint32_t)(uint16_t)lo[0] | ((uint32_t)(uint16_t)lo[1] << 16)),
             (int)((uint32_t)(uint16_t)lo[2] | ((uint32_t)(uint16_t)lo[3] << 16)),
             (int)((uint32_t)(uint16_t)hi[0] | ((uint32_t)(uint16_t)hi[1] << 16)),
             (int)((uint32_t)(uint16_t)hi[2] | ((uint32_t)(uint16_t)hi[3] << 16))};
}

// V operands are read VPRE MFMAs ahead of their use
constexpr int VPRE = 4;


// One piece of attn_wide_kernel's work: query tile `qlog` ((b, h, tile) in
// that order) over key tiles tb .. te - 1, in the LDS ring `lds` with the K
// block scales staged in `ks_l`. PIECE = false: the whole key range, the
// output stored; otherwise the unnormalized O (P = 2^(logit - m)), the running
// row maxima m and the row sums go to partial-result slot `slot`, in
// attn_piece's layout (the tiles are BQ rows).
template <int DT, int DP, bool PIECE>
__device__ __forceinline__ void wide_piece(const AttnArgs& p, uint8_t* lds, float* ks_l, int qlog, int tb_, int te_,
                                           int slot_) {
  using W = Wide<DP>;
  constexpr int ND = W::ND;
  static_assert(!PIECE || W::BQW == BQ, "partial results hold BQ-row tiles");
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, hf = lane >> 5, l32 = lane & 31;
  const int nqt = (p.Lq + W::BQW - 1) / W::BQW;
  const int qt = qlog % nqt, bh = qlog / nqt, b = bh / p.H, h = bh % p.H;
  const int ntiles = p.Lk64 / BKEY;
  // a whole query tile (PIECE = false) takes its key range as compile-time facts
  const int tb = PIECE ? tb_ : 0, te = PIECE ? te_ : ntiles, slot = PIECE ? slot_ : -1;
  // only the last key tile has keys past Lk
  const bool ragged = te == ntiles && p.Lk % BKEY != 0;

  // ---- DMA sources (byte offsets from the tile's first row). K: wave w
  // loads rows KRW w + lane / KC, physical chunk lane % KC, logical chunk
  // (lane % KC) ^ ((row >> KSH) % KC). V: rows VRW (w + NW u) + lane / (2 KC)
  // (u = 0, 1), physical chunk lane % (2 KC) in segment (lane % (2 KC)) / 4,
  // logical segment physical ^ ((row >> VSH) % VS), the chunk clamped to the
  // last one inside D (channels past D feed O rows that are never stored).
  const int8_t* kg = p.k8 + (int64_t)bh * p.Lk64 * DP;
  const uint16_t* vg = static_cast<const uint16_t*>(p.v) + b * p.vsb + h * p.vsh;
  const int krow = W::KRW * w + lane / W::KC;
  const uint32_t koff = (uint32_t)(krow * DP + 16 * ((lane % W::KC) ^ ((krow >> W::KSH) % W::KC)));
  int vrow[2], vcol[2];
  uint32_t voff[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    vrow[u] = W::VRW * (w + W::NW * u) + lane / (2 * W::KC);
    vcol[u] = min((lane % (2 * W::KC)) ^ (((vrow[u] >> W::VSH) % W::VS) << 2), p.D / 8 - 1) * 8;
    voff[u] = (uint32_t)(vrow[u] * (int)p.vsl + vcol[u]) * 2u;   // the host keeps p.vsl < WIDE_MAX_VSL
  }
  // tile `tile` into stage `st` ((tile - tb) % STAGES); past the piece's end
  // the source is its last tile again (in bounds; that data is never read)
  // the wave's DMA destinations in stage 0 (K, then V rows of u = 0, 1)
  const uint32_t lds0 = lds_addr(lds) + 1024 * w;
  auto issue = [&](int tile, int st) __attribute__((always_inline)) {
    const uint32_t sb = lds0 + st * W::WSTAGE;
    tile = min(tile, te - 1);
    dma16(reinterpret_cast<const uint8_t*>(kg) + tile * (BKEY * DP), koff, sb);
    const uint16_t* vt = vg + (int64_t)tile * BKEY * p.vsl;
    if (ragged && tile == ntiles - 1) {
      // keys past Lk read key Lk - 1 (their probabilities are 0; the values stay finite)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int key = min(tile * BKEY + vrow[u], p.Lk - 1) - tile * BKEY;
        dma16(vt, (uint32_t)(key * (int)p.vsl + vcol[u]) * 2u, sb + W::WK + 1024 * W::NW * u);
      }
    } else {
#pragma unroll
      for (int u = 0; u < 2; ++u) dma16(vt, voff[u], sb + W::WK + 1024 * W::NW * u);
    }
  };

  issue(tb, 0);
  issue(tb + 1, 1);
  issue(tb + 2, 2);
  // the piece's block scales into LDS (ordinary loads, waited for here,
  // before any DMA wait counts rely on the load order)
  for (int i = tb + t; i < te; i += W::NT) ks_l[i] = p.ks[(int64_t)bh * ntiles + i];

  // ---- Q: the wave's 32 rows, quantized per token into MFMA B operands
  v4i qf[ND];
  float cq;
  const int qrow = qt * W::BQW + w * 32 + l32;
  {
    const bool valid = qrow < p.Lq;
    const uint16_t* src = static_cast<const uint16_t*>(p.q) + b * p.qsb + (int64_t)(valid ? qrow : 0) * p.qsl + h * p.qsh;
    cq = quantize_q_row<DT, DP>(src, valid, p.D, hf, qf) * p.scale_log2;
  }

  // ---- operand offsets. K (A of S^T = K Q^T): row 32 kb + l32, logical chunk
  // 2 ks + hf, physical (2 ks + hf) ^ ((l32 >> KSH) % KC) (32 kb leaves the
  // swizzle unchanged).
  const int kx = (l32 >> W::KSH) % W::KC;
  int kfo[ND];
#pragma unroll
  for (int ks = 0; ks < ND; ++ks) kfo[ks] = l32 * DP + 16 * ((2 * ks + hf) ^ kx);
  // V^T (A of O^T = V^T P^T) by ds_read_tr16_b64: 16-lane group g16 of half hf
  // reads keys 16 kk + 4 hf + li / 4 (+ 8), channels 32 i + 16 g16 + 4 (li % 4);
  // such a key's row r has (r >> VSH) % VS = ((li / 4) >> VSH) % VS, so channel
  // block i sits at segment i ^ that
  const int li = lane & 15, g16 = (lane >> 4) & 1;
  const int vx = ((li >> 2) >> W::VSH) % W::VS;
  int vfo[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i) vfo[i] = (4 * hf + (li >> 2)) * W::VR + 64 * (i ^ vx) + 32 * g16 + 8 * (li & 3);

  float m = -INFINITY, lsum = 0.f;
  v16f o[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i) o[i] = v16f{0.f};
  v16i magic;
#pragma unroll
  for (int j = 0; j < 16; ++j) magic[j] = MAGIC_I;

  // Iteration `tile` (its stage st = (tile - tb) % STAGES, passed as a constant in
  // the unrolled loop so every LDS address is a lane base plus an immediate).
  // One barrier: before it each wave waits for its own loads of tile + 1;
  // after it tile + 1 is complete in LDS for every wave, and every wave is
  // done with tile - 1, whose stage receives tile + 3. Then the K operands of
  // tile + 1 and the first V operands of tile are read; most of the
  // exponentials of tile run while they land, then the QK^T MFMAs of tile + 1
  // into `nxt` interleave with the rest (at the last tile they recompute that
  // tile's scores, never used, so the phase stays branch-free); the lazy
  // maximum check (lazy_fixup: rescaling O when a probability may exceed
  // P_LIMIT); the PV MFMAs of tile, each reading the V operand VPRE MFMAs
  // ahead. TAIL: the ragged last tile.
  auto step = [&](int tile, int st, v16i (&cur)[2], v16i (&nxt)[2], auto tail) __attribute__((always_inline)) {
    constexpr bool TAIL = decltype(tail)::value;
    DC_ATTN_WAIT_VMCNT(WIDE_LOADS);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue(tile + 3, (st + 3) % ATTN_WIDE_STAGES);
    const uint8_t* sv = lds + st * W::WSTAGE + W::WK;
    v4i ka[2 * ND], va[4 * ND];
    k_operands<DP>(lds + ((st + 1) % ATTN_WIDE_STAGES) * W::WSTAGE, kfo, ka);
#pragma unroll
    for (int f = 0; f < VPRE; ++f) va[f] = v_operand<DP>(sv, vfo, f);
    __builtin_amdgcn_sched_barrier(0);
    const int key0 = tile * BKEY + 4 * hf;
    const float c = cq * ks_l[tile];
    uint32_t pk[2][8];
    float ts = 0.f;
    qk_mfma<DP>(ka, qf, magic, nxt);
    softmax_exp<DT, TAIL>(cur, key0, p.Lk, c, __builtin_fmaf(MAGIC_F, c, m), ts, pk);
    // UP of the ~96 VALU instructions of the exponentials first (the K
    // operand reads issued after the barrier land meanwhile, so the first
    // QK^T MFMA of tile + 1 does not hold up the in-order issue), then the
    // 2 ND MFMAs with the rest spread behind them. Measured at FLUX against
    // one MFMA then 12 VALU from the start: 2.7% faster per call, same bits;
    // 48 to 72 up front measure alike, all of it up front is slower. At
    // Dp = 64 (4 QK^T MFMAs) 72 up front measured 1.5% faster than 56 on
    // SD1.5's shape (40 alike; 24 and 96 slower).
    constexpr int UP = DP == 128 ? 56 : 72;
    __builtin_amdgcn_sched_group_barrier(0x002, UP, 0);
#pragma unroll
    for (int z = 0; z < 2 * ND; ++z) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, (96 - UP) / (2 * ND), 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    lazy_fixup<DT, DP, TAIL>(cur, key0, p.Lk, c, m, lsum, ts, o, pk);
    __builtin_amdgcn_sched_barrier(0);
    // PV: MFMA f consumes V operand f, read VPRE MFMAs earlier
#pragma unroll
    for (int f = 0; f < 4 * ND; ++f) {
      if (f + VPRE < 4 * ND) va[f + VPRE] = v_operand<DP>(sv, vfo, f + VPRE);
      const int kk = f / ND, kb = kk >> 1, j0 = 4 * (kk & 1);
      const v4i pf = {(int)pk[kb][j0], (int)pk[kb][j0 + 1], (int)pk[kb][j0 + 2], (int)pk[kb][j0 + 3]};
      o[f % ND] = mfma_pv<DT>(va[f], pf, o[f % ND]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  v16i sa[2], sb[2];
  // tile tb complete for every wave; the block scales are in LDS
  DC_ATTN_WAIT_VMCNT(2 * WIDE_LOADS);
  __syncthreads();
  {
    v4i ka[2 * ND];
    k_operands<DP>(lds, kfo, ka);
    qk_mfma<DP>(ka, qf, magic, sa);
  }
  // the last tile of a ragged key range runs masked, after the others; the
  // loop takes 4 tiles per trip (stages 0 .. 3 as constants), then 0 to 3 more
  const int nfull = ragged ? te - 1 : te;
  int tile = tb;
  for (; tile + 4 <= nfull; tile += 4) {
    step(tile, 0, sa, sb, std::false_type{});
    step(tile + 1, 1, sb, sa, std::false_type{});
    step(tile + 2, 2, sa, sb, std::false_type{});
    step(tile + 3, 3, sb, sa, std::false_type{});
  }
  // remaining tiles: stage (tile - tb) % 4 at run time, scores in sa
  for (; tile < nfull; ++tile) {
    step(tile, (tile - tb) % ATTN_WIDE_STAGES, sa, sb, std::false_type{});
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) sa[kb] = sb[kb];
  }
  if (ragged) step(tile, (tile - tb) % ATTN_WIDE_STAGES, sa, sb, std::true_type{});
  // no load may still be writing this workgroup's LDS when the piece ends
  DC_ATTN_WAIT_VMCNT(0);

  // ---- epilogue: O / l (each lane half summed its own keys)
  lsum += __shfl_xor(lsum, 32);
  if constexpr (PIECE) {
    float* part = p.part + (int64_t)slot * attn_part_floats<DP>();
    const int r = w * 32 + l32;
#pragma unroll
    for (int i = 0; i < ND; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<float4*>(part + r * DP + 32 * i + 8 * g + 4 * hf) =
            make_float4(o[i][4 * g], o[i][4 * g + 1], o[i][4 * g + 2], o[i][4 * g + 3]);
    if (hf == 0) {
      part[BQ * DP + r] = m;
      part[BQ * DP + BQ + r] = lsum;
    }
  } else if (qrow < p.Lq) {
    const float inv = 1.f / lsum;
    uint16_t* dst = static_cast<uint16_t*>(p.o) + b * p.osb + (int64_t)qrow * p.osl + h * p.osh;
#pragma unroll
    for (int i = 0; i < ND; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * i + 8 * g + 4 * hf;
        if (d >= p.D) continue;
        const uint32_t lo = f32_to_h16<DT>(o[i][4 * g] * inv) | (f32_to_h16<DT>(o[i][4 * g + 1] * inv) << 16);
        const uint32_t hi = f32_to_h16<DT>(o[i][4 * g + 2] * inv) | (f32_to_h16<DT>(o[i][4 * g + 3] * inv) << 16);
        *reinterpret_cast<uint2*>(dst + d) = make_uint2(lo, hi);
      }
  }
}

// Blocks 0 .. dp_blocks - 1 run whole query tiles (in XCD order). At Dp = 64
// the sk_blocks blocks after them run the stream-K share of the last sk_tiles
// query tiles as attn_kernel's do (pieces into partial slots 2 blk + piece,
// combined by attn_merge_kernel).
template <int DT, int DP>
__global__ void __launch_bounds__(Wide<DP>::NT, Wide<DP>::BLOCKS) attn_wide_kernel(AttnArgs p) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[ATTN_WIDE_STAGES * Wide<DP>::WSTAGE];
  __shared__ float ks_l[WIDE_MAX_TILES];   // the (b, h)'s K block scales
  if ((int)blockIdx.x < p.dp_blocks) {
    wide_piece<DT, DP, false>(p, lds, ks_l, xcd_order(blockIdx.x, p.dp_blocks), 0, 0, -1);
    return;
  }
  if constexpr (DP == 64) {
    const int ntiles = p.Lk64 / BKEY;
    const int blk = xcd_order(blockIdx.x - p.dp_blocks, p.sk_blocks);
    const int64_t units = (int64_t)p.sk_tiles * ntiles;
    const int64_t u_end = sk_first(blk + 1, units, p.sk_blocks);
    int64_t u = sk_first(blk, units, p.sk_blocks);
    for (int piece = 0; u < u_end; ++piece) {
      const int qi = (int)(u / ntiles), tb = (int)(u % ntiles);
      const int te = (int)min((int64_t)ntiles, tb + (u_end - u));
      // every wave is done with the previous piece's LDS stages and scales
      if (piece) __syncthreads();
      wide_piece<DT, DP, true>(p, lds, ks_l, p.dp_blocks + qi, tb, te, 2 * blk + piece);
      u += te - tb;
    }
  }
}
#undef DC_ATTN_WAIT_VMCNT

// ---------------------------------------------------------------- host

// Attention workgroups resident at once on the current device (occupancy x
// CUs, cached per device; concurrent first calls store the same value); 2 per
// CU on 256 CUs when no device answers.
template <int DT, int DP>
static int attn_slots() {
  static std::atomic<int> slots[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 512;
  int n = slots[dev].load(std::memory_order_relaxed);
  if (!n) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    // the kernel that runs the 128-query tiles: attn_wide_kernel at Dp = 64, attn_kernel at 128
    const void* fn = DP == 64 ? reinterpret_cast<const void*>(&attn_wide_kernel<DT, 64>)
                              : reinterpret_cast<const void*>(&attn_kernel<DT, DP>);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256, 0) != hipSuccess || per_cu <= 0) per_cu = 2;
    n = cus * per_cu;
    slots[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Work split (AttnArgs::dp_blocks / sk_blocks / sk_tiles). Query tiles fill
// whole rounds of `slots` workgroups data-parallel; when the last round would
// leave at least half the slots idle, its tiles' (query tile, key tile) units
// are shared evenly by up to `slots` stream-K workgroups instead (at least 16
// key tiles and an eighth of a query tile each). Measured on MI355X, a
// stream-K unit costs about 1.2 whole-tile units (each piece repeats the Q
// and first-tile prologue and stores its partial) and the merge about a
// tenth of a round, so a last round fuller than half gains nothing.
struct AttnPlan {
  int dp_blocks, sk_blocks, sk_tiles;
  bool wide;
};
static AttnPlan attn_plan(int64_t qtiles, int ntiles, int slots) {
  AttnPlan pl{(int)qtiles, 0, 0, false};
  if (ntiles < 32 || slots <= 0) return pl;
  const int64_t rounds = qtiles / slots, rest = qtiles % slots;
  if (rest == 0 || 2 * rest > slots) return pl;
  const int64_t units = rest * ntiles;
  // at least 16 key tiles and an eighth of a query tile per block
  const int64_t sk = std::min<int64_t>(slots, units / std::max(16, (ntiles + 7) / 8));
  if (sk <= 0) return pl;
  // a block's range touches at most two query tiles (two partial slots), and
  // a query tile is split into at most ATTN_MAX_PIECES pieces
  const int64_t longest = (units + sk - 1) / sk, shortest = units / sk;
  if (longest > ntiles || (ntiles + shortest - 1) / shortest + 1 > ATTN_MAX_PIECES) return pl;
  const double t_dp = (double)(rounds + 1), t_sk = (double)rounds + 1.2 * (double)units / ((double)sk * ntiles) + 0.1;
  if (t_sk > 0.95 * t_dp) return pl;
  pl.dp_blocks = (int)(rounds * slots);
  pl.sk_blocks = (int)sk;
  pl.sk_tiles = (int)rest;
  return pl;
}

// Compute units of the current device (cached per device; concurrent first
// calls store the same value); 256 when no device answers.
static int attn_cus() {
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

template <int DP>
static AttnPlan attn_plan_dp(int dtype, int B, int H, int Lq, int Lk) {
  const bool wide_ok = (Lk + BKEY - 1) / BKEY <= WIDE_MAX_TILES;
  if constexpr (DP == 128) {
    // attn_wide_kernel (whole 256-row query tiles, no stream-K split) when its
    // tiles fill at least one workgroup per CU; smaller grids keep the
    // 128-row tiles, which spread the work over twice the workgroups
    // (measured at 1 x 4 x 1024 x 1024: 34.5 us against 40 us)
    const int64_t wblocks = (int64_t)((Lq + Wide<128>::BQW - 1) / Wide<128>::BQW) * H * B;
    if (wide_ok && wblocks >= attn_cus()) return AttnPlan{(int)wblocks, 0, 0, true};
  }
  const int64_t qtiles = (int64_t)((Lq + BQ - 1) / BQ) * H * B;
  const int ntiles = (Lk + BKEY - 1) / BKEY;
  const int slots = dtype == DC_BF16 ? attn_slots<DC_BF16, DP>() : attn_slots<DC_F16, DP>();
  AttnPlan pl = attn_plan(qtiles, ntiles, slots);
  if constexpr (DP == 64) {
    // at Dp = 64 attn_wide_kernel runs the same 128-row query tiles and
    // stream-K pieces as attn_kernel (two workgroups per CU)
    static_assert(Wide<64>::BQW == BQ, "the Dp = 64 wide tiles are attn_kernel's query tiles");
    if (wide_ok) pl.wide = true;
  }
  return pl;
}

struct WsLayout {
  size_t k8, ks, kpart, ksum, part, total;
};

static size_t up256(size_t x) { return (x + 255) / 256 * 256; }

// sk_blocks: stream-K workgroups of the plan (two partial-result slots each)
static WsLayout ws_layout(int B, int H, int Lk, int D, int sk_blocks) {
  const size_t bh = (size_t)B * H;
  const size_t dp = D <= 64 ? 64 : 128;
  const size_t lk = ((size_t)Lk + BKEY - 1) / BKEY * BKEY;
  const size_t nwin = ((size_t)Lk + WIN - 1) / WIN;
  WsLayout w{};
  size_t off = 0;
  w.k8 = off; off += up256(bh * lk * dp);
  w.ks = off; off += up256(bh * (lk / BKEY) * 4);
  w.kpart = off; off += up256(bh * nwin * D * 4);
  w.ksum = off; off += up256(bh * D * 4);
  w.part = off; off += up256((size_t)2 * sk_blocks * (dp == 64 ? attn_part_floats<64>() : attn_part_floats<128>()) * 4);
  w.total = off;
  return w;
}

template <int DT, int DP>
static int launch_attn(AttnArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((kstats_kernel<DT>), dim3(a.nwin, a.H, a.B), dim3(256), 0, st, a);
  if (int e = launch_status("kstats_kernel")) return e;
  hipLaunchKernelGGL((kquant_kernel<DT, DP>), dim3((a.Lk64 / BKEY + KQ_BLOCKS - 1) / KQ_BLOCKS, a.H, a.B), dim3(256),
                     0, st, a);
  if (int e = launch_status("kquant_kernel")) return e;
  if (a.wide) {
    hipLaunchKernelGGL((attn_wide_kernel<DT, DP>), dim3((unsigned)(a.dp_blocks + a.sk_blocks)), dim3(Wide<DP>::NT), 0,
                       st, a);
    if (int e = launch_status("attn_wide_kernel")) return e;
  } else {
    hipLaunchKernelGGL((attn_kernel<DT, DP>), dim3((unsigned)(a.dp_blocks + a.sk_blocks)), dim3(256), 0, st, a);
    if (int e = launch_status("attn_kernel")) return e;
  }
  if (a.sk_blocks == 0) return DC_OK;
  hipLaunchKernelGGL((attn_merge_kernel<DT, DP>), dim3((unsigned)a.sk_tiles), dim3(256), 0, st, a);
  return launch_status("attn_merge_kernel");
}

// Shared argument checks; fills the strides and shapes of `a`.
static int check_args(const void* q, int dtype, int B, int H, int Lq, int D, const int64_t* q_strides, AttnArgs& a) {
  if (dtype != DC_F16 && dtype != DC_BF16) return fail(DC_EINVAL, "int8 attention: dtype must be DC_F16 or DC_BF16");
  if (B <= 0 || H <= 0 || Lq <= 0) return fail(DC_EINVAL, "int8 attention: empty attention input");
  if (D <= 0 || D > 128 || D % 8) return fail(DC_EUNSUPPORTED, "int8 attention: head dim must be a multiple of 8, <= 128");
  if (!q || !q_strides) return fail(DC_EINVAL, "int8 attention: null pointer");
  if (!aligned16(q)) return fail(DC_EUNSUPPORTED, "int8 attention: q must be 16-byte aligned");
  for (int i = 0; i < 3; ++i)
    if (q_strides[i] % 8 || q_strides[i] < 0)
      return fail(DC_EUNSUPPORTED, "int8 attention: (B, L, H) strides must be non-negative multiples of 8");
  if ((int64_t)B * H * ((Lq + BQ - 1) / BQ) > 0x7fffffff || (int64_t)Lq + BQ > 0x7fffffff)
    return fail(DC_EINVAL, "int8 attention: problem too large");
  a.q = q; a.B = B; a.H = H; a.Lq = Lq; a.D = D;
  a.qsb = q_strides[0]; a.qsl = q_strides[1]; a.qsh = q_strides[2];
  return DC_OK;
}

extern "C" size_t dc_int8_attn_workspace_bytes(int B, int H, int Lq, int Lk, int D) {
  if (B <= 0 || H <= 0 || Lq <= 0 || Lk <= 0 || D <= 0 || D > 128) return 0;
  // room for the larger of the two dtypes' plans
  size_t bytes = 0;
  for (int dt : {DC_F16, DC_BF16}) {
    const AttnPlan pl = D <= 64 ? attn_plan_dp<64>(dt, B, H, Lq, Lk) : attn_plan_dp<128>(dt, B, H, Lq, Lk);
    bytes = std::max(bytes, ws_layout(B, H, Lk, D, pl.sk_blocks).total);
  }
  return bytes;
}

extern "C" int dc_int8_attn_plan(int dtype, int B, int H, int Lq, int Lk, int D, int* dp_tiles, int* sk_blocks,
                                 int* sk_tiles) {
  clear_error();
  if (dtype != DC_F16 && dtype != DC_BF16) return fail(DC_EINVAL, "dc_int8_attn_plan: dtype must be DC_F16 or DC_BF16");
  if (B <= 0 || H <= 0 || Lq <= 0 || Lk <= 0 || D <= 0 || D > 128)
    return fail(DC_EINVAL, "dc_int8_attn_plan: bad shape");
  if (!dp_tiles || !sk_blocks || !sk_tiles) return fail(DC_EINVAL, "dc_int8_attn_plan: null pointer");
  const AttnPlan pl = D <= 64 ? attn_plan_dp<64>(dtype, B, H, Lq, Lk) : attn_plan_dp<128>(dtype, B, H, Lq, Lk);
  *dp_tiles = pl.dp_blocks;
  *sk_blocks = pl.sk_blocks;
  *sk_tiles = pl.sk_tiles;
  return DC_OK;
}

// Shared body of dc_int8_attn_fwd and dc_int8_attn_fwd_noalloc: checks,
// workspace carve-up and launches. `who` names the entry point in messages.
static int attn_fwd(const void* q, const void* k, const void* v, void* o, int dtype, int B, int H, int Lq, int Lk,
                    int D, const int64_t q_strides[3], const int64_t k_strides[3], const int64_t v_strides[3],
                    const int64_t o_strides[3], float sm_scale, void* workspace, size_t ws_bytes, void* stream,
                    const char* who) {
  AttnArgs a{};
  if (int e = check_args(q, dtype, B, H, Lq, D, q_strides, a)) return e;
  if (Lk <= 0) { set_error("%s: empty attention input", who); return DC_EINVAL; }
  if (!k || !v || !o || !k_strides || !v_strides || !o_strides) { set_error("%s: null pointer", who); return DC_EINVAL; }
  if (!aligned16(k) || !aligned16(v) || !aligned16(o)) {
    set_error("%s: q, k, v, o must be 16-byte aligned", who);
    return DC_EUNSUPPORTED;
  }
  for (int i = 0; i < 3; ++i)
    if (k_strides[i] % 8 || v_strides[i] % 8 || o_strides[i] % 8 || k_strides[i] < 0 || v_strides[i] < 0 ||
        o_strides[i] < 0) {
      set_error("%s: (B, L, H) strides must be non-negative multiples of 8", who);
      return DC_EUNSUPPORTED;
    }
  if ((int64_t)Lk + WIN > 0x7fffffff) { set_error("%s: problem too large", who); return DC_EINVAL; }
  AttnPlan pl = D <= 64 ? attn_plan_dp<64>(dtype, B, H, Lq, Lk) : attn_plan_dp<128>(dtype, B, H, Lq, Lk);
  if (pl.wide && v_strides[1] >= WIDE_MAX_VSL) {
    // attn_wide_kernel addresses a tile's 64 V rows with 32-bit offsets; a
    // longer V row stride takes the 128-query kernel (64-bit offsets) with
    // whole query tiles, which needs no more workspace than the wide plan
    pl = AttnPlan{(int)((int64_t)((Lq + BQ - 1) / BQ) * H * B), 0, 0, false};
  }
  const WsLayout w = ws_layout(B, H, Lk, D, pl.sk_blocks);
  if (!workspace || ws_bytes < w.total) {
    set_error("%s: workspace too small (%zu bytes, this call needs %zu)", who, ws_bytes, w.total);
    return DC_EWORKSPACE;
  }
  if (!aligned16(workspace)) { set_error("%s: workspace must be 16-byte aligned", who); return DC_EWORKSPACE; }
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  a.k = k; a.v = v; a.o = o;
  a.k8 = reinterpret_cast<int8_t*>(ws + w.k8);
  a.ks = reinterpret_cast<float*>(ws + w.ks);
  a.kpart = reinterpret_cast<float*>(ws + w.kpart);
  a.ksum = reinterpret_cast<float*>(ws + w.ksum);
  a.part = reinterpret_cast<float*>(ws + w.part);
  a.dp_blocks = pl.dp_blocks;
  a.sk_blocks = pl.sk_blocks;
  a.sk_tiles = pl.sk_tiles;
  a.wide = pl.wide ? 1 : 0;
  a.Lk = Lk;
  a.Lk64 = (Lk + BKEY - 1) / BKEY * BKEY;
  a.nwin = (Lk + WIN - 1) / WIN;
  a.ksb = k_strides[0]; a.ksl = k_strides[1]; a.ksh = k_strides[2];
  a.vsb = v_strides[0]; a.vsl = v_strides[1]; a.vsh = v_strides[2];
  a.osb = o_strides[0]; a.osl = o_strides[1]; a.osh = o_strides[2];
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == DC_BF16) return D <= 64 ? launch_attn<DC_BF16, 64>(a, st) : launch_attn<DC_BF16, 128>(a, st);
  return D <= 64 ? launch_attn<DC_F16, 64>(a, st) : launch_attn<DC_F16, 128>(a, st);
}

// ---------------------------------------------------------------- no-allocation entry point

// Scratch of dc_int8_attn_fwd_noalloc: a file-scope device array (each GPU
// the library runs on holds its own copy, of DC_ATTN_NOALLOC_MAX_BYTES, until
// the process ends). Its name is a host-side stand-in, not a device address:
// host code uses only the per-device pointer hipGetSymbolAddress returns,
// looked up once per device with that device current.
static __device__ __align__(256) uint8_t scratch[DC_ATTN_NOALLOC_MAX_BYTES];

constexpr int SCRATCH_DEVICES = 64;
static std::once_flag scratch_once[SCRATCH_DEVICES];
static void* scratch_ptr[SCRATCH_DEVICES];
static hipError_t scratch_err[SCRATCH_DEVICES];

// This device's copy of `scratch` (looked up on the first call per device).
static int device_scratch(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= SCRATCH_DEVICES)
    return fail(DC_EHIP, "dc_int8_attn_fwd_noalloc: no current HIP device");
  std::call_once(scratch_once[dev], [dev] {
    void* p = nullptr;
    scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    scratch_ptr[dev] = p;
  });
  if (scratch_err[dev] != hipSuccess || !scratch_ptr[dev]) {
    set_error("dc_int8_attn_fwd_noalloc: hipGetSymbolAddress of the scratch array failed: %s",
              hipGetErrorString(scratch_err[dev]));
    return DC_EHIP;
  }
  *out = scratch_ptr[dev];
  return DC_OK;
}

}  // namespace dc

using namespace dc;

extern "C" int dc_int8_attn_fwd(const void* q, const void* k, const void* v, void* o, int dtype, int B, int H, int Lq,
                                int Lk, int D, const int64_t q_strides[3], const int64_t k_strides[3],
                                const int64_t v_strides[3], const int64_t o_strides[3], float sm_scale,
                                void* workspace, size_t ws_bytes, void* stream) {
  clear_error();
  return attn_fwd(q, k, v, o, dtype, B, H, Lq, Lk, D, q_strides, k_strides, v_strides, o_strides, sm_scale, workspace,
                  ws_bytes, stream, "dc_int8_attn_fwd");
}

extern "C" int dc_int8_attn_fwd_noalloc(const void* q, const void* k, const void* v, void* o, int dtype, int B, int H,
                                        int Lq, int Lk, int D, const int64_t q_strides[3],
                                        const int64_t k_strides[3], const int64_t v_strides[3],
                                        const int64_t o_strides[3], float sm_scale, void* stream) {
  clear_error();
  if (dtype != DC_F16 && dtype != DC_BF16)
    return fail(DC_EINVAL, "dc_int8_attn_fwd_noalloc: dtype must be DC_F16 or DC_BF16");
  if (B <= 0 || H <= 0 || Lq <= 0 || Lk <= 0) return fail(DC_EINVAL, "dc_int8_attn_fwd_noalloc: empty attention input");
  if (D <= 0 || D > 128 || D % 8)
    return fail(DC_EUNSUPPORTED, "dc_int8_attn_fwd_noalloc: head dim must be a multiple of 8, <= 128");
  if ((int64_t)B * H * ((Lq + BQ - 1) / BQ) > 0x7fffffff || (int64_t)Lq + BQ > 0x7fffffff ||
      (int64_t)Lk + WIN > 0x7fffffff)
    return fail(DC_EINVAL, "dc_int8_attn_fwd_noalloc: problem too large");
  const AttnPlan pl = D <= 64 ? attn_plan_dp<64>(dtype, B, H, Lq, Lk) : attn_plan_dp<128>(dtype, B, H, Lq, Lk);
  const size_t need = ws_layout(B, H, Lk, D, pl.sk_blocks).total;
  if (need > DC_ATTN_NOALLOC_MAX_BYTES) {
    set_error("dc_int8_attn_fwd_noalloc: this call needs %zu bytes of scratch, more than the %zu it holds; use "
              "dc_int8_attn_fwd with a workspace", need, (size_t)DC_ATTN_NOALLOC_MAX_BYTES);
    return DC_EWORKSPACE;
  }
  void* ws = nullptr;
  if (int e = device_scratch(&ws)) return e;
  return attn_fwd(q, k, v, o, dtype, B, H, Lq, Lk, D, q_strides, k_strides, v_strides, o_strides, sm_scale, ws,
                  DC_ATTN_NOALLOC_MAX_BYTES, stream, "dc_int8_attn_fwd_noalloc");
}

extern "C" int dc_int8_attn_quantize_q(const void* q, int dtype, int B, int H, int Lq, int D,
                                       const int64_t q_strides[3], int8_t* q8, float* qs, void* stream) {
  clear_error();
  AttnArgs a{};
  if (int e = check_args(q, dtype, B, H, Lq, D, q_strides, a)) return e;
  if (!q8 || !qs) return fail(DC_EINVAL, "dc_int8_attn_quantize_q: null output");
  if (!aligned16(q8)) return fail(DC_EUNSUPPORTED, "dc_int8_attn_quantize_q: q8 must be 16-byte aligned");
  const int lq32 = (Lq + 31) / 32 * 32;
  const dim3 grid(lq32 / 32, B * H);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == DC_BF16) {
    if (D <= 64) hipLaunchKernelGGL((qquant_kernel<DC_BF16, 64>), grid, dim3(64), 0, st, a, q8, qs, lq32);
    else hipLaunchKernelGGL((qquant_kernel<DC_BF16, 128>), grid, dim3(64), 0, st, a, q8, qs, lq32);
  } else {
    if (D <= 64) hipLaunchKernelGGL((qquant_kernel<DC_F16, 64>), grid, dim3(64), 0, st, a, q8, qs, lq32);
    else hipLaunchKernelGGL((qquant_kernel<DC_F16, 128>), grid, dim3(64), 0, st, a, q8, qs, lq32);
  }
  return launch_status("qquant_kernel");
}
