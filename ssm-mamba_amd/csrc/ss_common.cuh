#include <algorithm>
#include <type_traits>
// Device helpers shared by the selective-scan and state-update kernels (gfx950).
//
// Element types: the streamed tensors (u, delta, z, out, dout, du, ddelta, dz,
// B, C, dB, dC) are either fp32 or bf16; all arithmetic is fp32.  Parameters
// (A, D, delta_bias), states and state gradients are fp32.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

namespace ssm {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------- bf16 / fp32 I/O

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// one stored element to fp32
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(__hip_bfloat16 x) {
  return __uint_as_float((uint32_t)__builtin_bit_cast(uint16_t, x) << 16);
}

typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
typedef float f32x2_v __attribute__((ext_vector_type(2)));

// Two floats to bf16, round-to-nearest-even, lo in bits 0-15: one
// v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_v v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_v));
}

template <typename T> struct Elem;

template <> struct Elem<float> {
  static constexpr int kVec = 4;  // elements per 128-bit access
  __device__ static __forceinline__ float load1(const float* p) { return *p; }
  __device__ static __forceinline__ void store1(float* p, float v) { *p = v; }
  // 128-bit load of kVec elements
  __device__ static __forceinline__ void loadv(const float* p, float (&v)[4]) {
    float4 x = *reinterpret_cast<const float4*>(p);
    v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
  }
  __device__ static __forceinline__ void storev(float* p, const float (&v)[4]) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  }
  // 4 consecutive elements (16 B for fp32)
  __device__ static __forceinline__ void load4(const float* p, float (&v)[4]) { loadv(p, v); }
};

template <> struct Elem<__hip_bfloat16> {
  static constexpr int kVec = 8;
  using T = __hip_bfloat16;
  __device__ static __forceinline__ float load1(const T* p) {
    return __uint_as_float((uint32_t)(*reinterpret_cast<const uint16_t*>(p)) << 16);
  }
  __device__ static __forceinline__ void store1(T* p, float v) { *p = __float2bfloat16(v); }
  __device__ static __forceinline__ void loadv(const T* p, float (&v)[8]) {
    uint4 x = *reinterpret_cast<const uint4*>(p);
    v[0] = bf16_lo(x.x); v[1] = bf16_hi(x.x); v[2] = bf16_lo(x.y); v[3] = bf16_hi(x.y);
    v[4] = bf16_lo(x.z); v[5] = bf16_hi(x.z); v[6] = bf16_lo(x.w); v[7] = bf16_hi(x.w);
  }
  __device__ static __forceinline__ void storev(T* p, const float (&v)[8]) {
    uint4 x;
    x.x = pack_bf16x2(v[0], v[1]); x.y = pack_bf16x2(v[2], v[3]);
    x.z = pack_bf16x2(v[4], v[5]); x.w = pack_bf16x2(v[6], v[7]);
    *reinterpret_cast<uint4*>(p) = x;
  }
  // 4 consecutive elements (8 B for bf16)
  __device__ static __forceinline__ void load4(const T* p, float (&v)[4]) {
    uint2 x = *reinterpret_cast<const uint2*>(p);
    v[0] = bf16_lo(x.x); v[1] = bf16_hi(x.x); v[2] = bf16_lo(x.y); v[3] = bf16_hi(x.y);
  }
};

// ---------------------------------------------------------------- math

// 2^x on the transcendental unit (v_exp_f32).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// The carry through a run of segment summaries for one (batch row b, channel
// ch, state n): x <- exp2(A2 dt_k) x + g_k for k = k_first, k_first + step,
// ... (count terms), with dt_k = dtp[(k * batch + b) * Dm + ch] and g_k =
// gp[((k * batch + b) * N + n) * Dm + ch].  The loads are issued eight at a
// time ahead of their multiply-adds, so a long run waits for memory once per
// eight terms instead of once per term; the arithmetic and its order are
// those of the plain loop.
__device__ __forceinline__ float fold_carry(float x, float A2, const float* __restrict__ dtp,
                                            const float* __restrict__ gp, int k_first, int step,
                                            int count, int batch, int b, int Dm, int N, int n,
                                            int ch) {
  for (int c0 = 0; c0 < count; c0 += 8) {
    float dt[8], g[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int c = min(c0 + u, count - 1);
      const size_t kb = (size_t)(k_first + step * c) * batch + b;
      dt[u] = dtp[kb * Dm + ch];
      g[u] = gp[(kb * N + n) * Dm + ch];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (c0 + u < count) x = fmaf(fast_exp2(A2 * dt[u]), x, g[u]);
  }
  return x;
}
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// log1p(e) for 0 <= e <= 1.  w = 1 + e rounds away c = (w - 1) - e, which is
// exact (Sterbenz: w - 1 and e are within a factor of two of each other, or
// w == 1 and c = -e); then log1p(e) = log(w) + log(1 - c / w), and
// log(1 - c / w) = -c / w to within c^2 / 2, and 1 / w = 2 - w to within
// (w - 1)^2.  With |c| <= 2^-24 and |c| <= e, both dropped terms stay below
// 2^-24 relative to log1p(e): no reciprocal and no select are needed.
__device__ __forceinline__ float log1p_pos(float e) {
  const float w = 1.0f + e;
  const float c = (w - 1.0f) - e;
  return fmaf(fast_log2(w), kLn2, -c * (2.0f - w));
}

// softplus with the reference threshold: x <= 20 ? log1p(exp(x)) : x.
// Evaluated as max(x,0) + log1p(exp(-|x|)), which is the same function and keeps
// exp's argument non-positive.  The threshold needs no select: above 20,
// exp(-|x|) < 2.1e-9 rounds 1 + e to 1, log1p_pos returns e itself, and x + e
// rounds to x (half an ulp of x is 9.5e-7 there); infinities and NaN pass
// through as in the reference.
__device__ __forceinline__ float softplus_t20(float x) {
  const float e = fast_exp2(-fabsf(x) * kLog2e);
  return fmaxf(x, 0.0f) + log1p_pos(e);
}

__device__ __forceinline__ float sigmoidf_fast(float x) {
  return fast_rcp(1.0f + fast_exp2(-x * kLog2e));
}

// softplus and its derivative (threshold 20) from one exponential:
// e = exp(-|x|), sigmoid(x) = x >= 0 ? 1 / (1 + e) : e / (1 + e).
__device__ __forceinline__ void softplus_and_grad_t20(float x, float& sp, float& sg) {
  const float e = fast_exp2(-fabsf(x) * kLog2e);
  const float r = fast_rcp(1.0f + e);
  sp = fmaxf(x, 0.0f) + log1p_pos(e);  // equals x above 20 (see softplus_t20)
  sg = x > 20.0f ? 1.0f : (x >= 0.0f ? r : e * r);
}

// d softplus/dx with the reference threshold (sigmoid below 20, 1 above).
__device__ __forceinline__ float softplus_grad_t20(float x) {
  return x > 20.0f ? 1.0f : sigmoidf_fast(x);
}

// ---------------------------------------------------------------- wave64 primitives

// DPP controls (GCN/CDNA encoding)
constexpr int kDppRowRor8 = 0x128;
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppQuadXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppQuadXor1 = 0xB1;  // quad_perm [1,0,3,2]

template <int kCtrl>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kCtrl, 0xF, 0xF, true));
}

// One reduce-scatter level that folds lane bit `kBit` using a DPP pattern whose
// partner differs from the lane in that bit.  p, q are the two halves of a
// pair of values; the lane keeps the half selected by its bit and receives the
// partner's copy of the same half.
template <int kCtrl>
__device__ __forceinline__ float rs_fold(float p, float q, bool bit) {
  float keep = bit ? q : p;
  float send = bit ? p : q;
  return keep + dpp_mov<kCtrl>(send);
}

// Reduce-scatter of K values held by every lane of a wave64: afterwards the
// sum over the 64 lanes of value index (lane * K/64 + j) is in v[j] of `lane`,
// for j < K/64.  Cost ~2.2 VALU per input value (permlane32/16 swaps for the
// two upper levels, DPP for the four lower ones).
template <int K>
__device__ __forceinline__ void wave_reduce_scatter(float (&v)[K], int lane) {
  static_assert(K >= 64 && (K & (K - 1)) == 0, "K must be a power of two >= 64");
#pragma unroll
  for (int i = 0; i < K / 2; ++i) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[i + K / 2]),
                                              false, false);
    v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int i = 0; i < K / 4; ++i) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]), __float_as_uint(v[i + K / 4]),
                                              false, false);
    v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  const bool b3 = lane & 8, b2 = lane & 4, b1 = lane & 2, b0 = lane & 1;
#pragma unroll
  for (int i = 0; i < K / 8; ++i) v[i] = rs_fold<kDppRowRor8>(v[i], v[i + K / 8], b3);
#pragma unroll
  for (int i = 0; i < K / 16; ++i) v[i] = rs_fold<kDppRowHalfMirror>(v[i], v[i + K / 16], b2);
#pragma unroll
  for (int i = 0; i < K / 32; ++i) v[i] = rs_fold<kDppQuadXor2>(v[i], v[i + K / 32], b1);
#pragma unroll
  for (int i = 0; i < K / 64; ++i) v[i] = rs_fold<kDppQuadXor1>(v[i], v[i + K / 64], b0);
}

// Sum over the 64 lanes of 16 values per lane: afterwards v[0] of lane l
// holds the total of value index l >> 2 (the four lanes of a quad hold the
// same total).  Four reduce-scatter levels (lane bits 5..2) then two
// all-reduce levels inside the quad; ~2.2 VALU per input value.
__device__ __forceinline__ void wave_reduce16(float (&v)[16], int lane) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[i + 8]),
                                              false, false);
    v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]), __float_as_uint(v[i + 4]),
                                              false, false);
    v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  const bool b3 = lane & 8, b2 = lane & 4;
#pragma unroll
  for (int i = 0; i < 2; ++i) v[i] = rs_fold<kDppRowRor8>(v[i], v[i + 2], b3);
  v[0] = rs_fold<kDppRowHalfMirror>(v[0], v[1], b2);
  v[0] += dpp_mov<kDppQuadXor1>(v[0]);
  v[0] += dpp_mov<kDppQuadXor2>(v[0]);
}

// ---------------------------------------------------------------- row broadcasts
// A "block register" holds 16 wave-uniform values, value k in lane k of every
// 16-lane row (lane l holds value l & 15).  DPP row_newbcast:k (gfx90a and
// later) reads value k in every lane as an instruction operand, so a block
// of 16 values costs one VGPR and one 4-byte load per lane instead of 16
// registers or 128-bit broadcast LDS reads.  k must fold to a constant.
#define SSM_ROW16(X) X(0) X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8) X(9) X(10) X(11) X(12) X(13) X(14) X(15)

// value k * x: the compiler folds the DPP move into v_mul_f32_dpp
__device__ __forceinline__ float bc_mul(int k, float blk, float x) {
  int v = 0;
  switch (k) {
#define SSM_BC_MUL(n) \
  case n: v = __builtin_amdgcn_update_dpp(0, __float_as_int(blk), 0x150 + n, 0xF, 0xF, true); break;
    SSM_ROW16(SSM_BC_MUL)
#undef SSM_BC_MUL
  }
  return __int_as_float(v) * x;
}

// acc + value k * x as one v_fmac_f32_dpp.  The compiler does not fold a DPP
// operand into v_fmac on this architecture, hence the inline instruction.
// A DPP read of blk needs two wait states after a VALU write of blk, which the
// compiler cannot see inside the asm; blk is a block register read from LDS
// and never written by a VALU instruction, so none are inserted here (an
// s_nop per use cost the backward 2%).  tests/test_dpp_hazards.py checks the
// compiled kernels for any VALU write of a DPP source within two wait states.
__device__ __forceinline__ float bc_fmac(int k, float acc, float blk, float x) {
  switch (k) {
#define SSM_BC_FMAC(n)                                                                         \
  case n:                                                                                     \
    asm("v_fmac_f32_dpp %0, %1, %2 row_newbcast:" #n                                           \
        " row_mask:0xf bank_mask:0xf bound_ctrl:1"                                             \
        : "+v"(acc)                                                                           \
        : "v"(blk), "v"(x));                                                                  \
    break;
    SSM_ROW16(SSM_BC_FMAC)
#undef SSM_BC_FMAC
  }
  return acc;
}

// Sum over groups of kW consecutive lanes (kW power of two <= 64); every lane
// of a group gets the group sum.
template <int kW>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int m = 1; m < kW; m <<= 1) v += __shfl_xor(v, m, 64);
  return v;
}

__device__ __forceinline__ int wave_id_uniform() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

}  // namespace ssm
