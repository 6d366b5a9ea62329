// RMSNorm over the channel axis of channel-major activations (batch, C, L),
// for gfx950:
//
//   out[b, c, t] = x[b, c, t] * rsqrt(mean_c x[b, c, t]^2 + eps) * (1 + w[c])
//
// the reference's RMSNorm (modules/rms_norm.py:11-31: fp32 statistics, scale
// 1 + weight, result cast back to the input type) applied to the layout the
// scan streams, so the Mamba stack needs no (B, L, C) <-> (B, C, L) copies.
//
// A workgroup owns kPos positions of one batch row and all C channels, so the
// statistics need no second kernel.  Its lanes split into rows of kPos / kPL
// lanes, each lane holding kPL adjacent positions: one wave load covers
// 64 * kPL / kPos channel rows of kPos contiguous positions, and the 16 waves
// interleave over the channel rows.  Pass 1 accumulates x^2 per position;
// the rows of a wave are combined with lane shuffles and the waves through
// LDS.  Pass 2 writes the scaled result, taking a lane's first kHold rows
// from registers and re-reading the rest (L2-resident: a workgroup's tile is
// C * kPos elements).
//
// Small tiles keep the machine full at the model's shapes (batch 4 x 2048
// positions is 8192 positions: 32-position tiles give 256 workgroups).  A
// tile narrower than a 128-byte line shares its lines with its neighbours;
// the blockIdx -> tile map puts the workgroups that share a line on one XCD
// (workgroup g runs on XCD g % 8), so each line is fetched from HBM once into
// that XCD's L2.
#include "ss_common.cuh"
#include "ss_prof.h"

namespace ssm {

namespace {

constexpr int kNormThreads = 1024;
constexpr int kNormWaves = kNormThreads / 64;
constexpr int kNormXcds = 8;

template <typename T>
struct Pair;

template <>
struct Pair<float> {
  __device__ static __forceinline__ float2 load(const float* p) {
    return *reinterpret_cast<const float2*>(p);
  }
  __device__ static __forceinline__ void store(float* p, float a, float b) {
    *reinterpret_cast<float2*>(p) = make_float2(a, b);
  }
};

template <>
struct Pair<__hip_bfloat16> {
  __device__ static __forceinline__ float2 load(const __hip_bfloat16* p) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
    return make_float2(bf16_lo(w), bf16_hi(w));
  }
  __device__ static __forceinline__ void store(__hip_bfloat16* p, float a, float b) {
    *reinterpret_cast<uint32_t*>(p) = pack_bf16x2(a, b);
  }
};

// Channel rows per lane kept in registers between the two passes (the rest
// are re-read from L2, kBatch rows at a time): 16 cover d_model 1024 whole.
constexpr int kHold = 16;
constexpr int kBatch = 8;

// kPL = 2 and kPair: L even and rows 4-byte (bf16) / 8-byte (fp32) aligned,
// so a lane's two positions load and store as one element pair.  kShare:
// tiles sharing a 128-byte line (1, 2 or 4).
template <typename T, int kPos, int kPL, bool kPair, int kShare>
__global__ __launch_bounds__(kNormThreads) void rms_norm_cm_kernel(
    const T* __restrict__ x, const T* __restrict__ w, float eps, T* __restrict__ out, int C, int L,
    int tiles_per_row, int ntiles) {
  constexpr int kLPR = kPos / kPL;     // lanes per channel row
  constexpr int kRPL = 64 / kLPR;      // channel rows per wave load
  static_assert(kLPR * kRPL == 64 && kPL >= 1 && kPL <= 2, "tile shape");
  __shared__ float s_ss[kNormWaves][kPos];
  // blockIdx -> tile: the kShare tiles of one line go to workgroups g, g + 8,
  // ... (same XCD)
  const int g = blockIdx.x;
  const int grp = g / (kNormXcds * kShare);
  const int within = g % (kNormXcds * kShare);
  const int line = grp * kNormXcds + within % kNormXcds;
  const int tile = line * kShare + within / kNormXcds;
  if (tile >= ntiles) return;  // whole workgroup, before any barrier
  const int b = tile / tiles_per_row;
  const int t0 = (tile - b * tiles_per_row) * kPos;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int prow = lane % kLPR;  // position slot
  const int crow = lane / kLPR;  // channel row slot in a wave load
  const int t = t0 + kPL * prow;
  const bool ok0 = t < L, ok1 = kPL == 2 && t + 1 < L;
  const T* __restrict__ xb = x + (size_t)b * C * L;
  T* __restrict__ ob = out + (size_t)b * C * L;
  constexpr int kStride = kNormWaves * kRPL;  // channel rows per workgroup sweep
  const int c_first = wave * kRPL + crow;

  // Loads read clamped (always valid) addresses and out-of-range values are
  // zeroed afterwards: all loads of a batch issue first, then pass through an
  // empty asm (so the compiler cannot turn the zeroing back into a branch
  // around the load, where it would be waited for at once), then are masked.
  // A pair load at t <= L - 2 stays aligned (t and L even).
  const int tp = kPair ? min(t, L - 2) : min(t, L - 1);
  const int tq = min(t + 1, L - 1);
  auto raw2 = [&](int c) -> float2 {
    const T* p = xb + (size_t)min(c, C - 1) * L;
    if constexpr (kPL == 1) {
      return make_float2(Elem<T>::load1(p + tp), 0.f);
    } else if constexpr (kPair) {
      return Pair<T>::load(p + tp);
    } else {
      return make_float2(Elem<T>::load1(p + tp), Elem<T>::load1(p + tq));
    }
  };
  auto mask2 = [&](int c, float2 v) -> float2 {
    const bool okc = c < C;
    return make_float2(okc && ok0 ? v.x : 0.f, okc && ok1 ? v.y : 0.f);
  };
  auto scale_of = [&](int c) { return 1.0f + Elem<T>::load1(w + min(c, C - 1)); };
  auto pin = [](float2& v) { asm volatile("" : "+v"(v.x), "+v"(v.y)); };

  // the first kHold channel rows of a lane stay in registers for pass 2, with
  // their weights
  float2 held[kHold];
  float gw_held[kHold];
#pragma unroll
  for (int i = 0; i < kHold; ++i) {
    held[i] = raw2(c_first + i * kStride);
    gw_held[i] = scale_of(c_first + i * kStride);
  }
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int i = 0; i < kHold; ++i) pin(held[i]);
#pragma unroll
  for (int i = 0; i < kHold; ++i) {
    held[i] = mask2(c_first + i * kStride, held[i]);
    s0 = fmaf(held[i].x, held[i].x, s0);
    s1 = fmaf(held[i].y, held[i].y, s1);
  }
  // the remaining rows, kBatch loads in flight per lane (rows past C read 0)
  for (int c0 = c_first + kHold * kStride; c0 < C; c0 += kBatch * kStride) {
    float2 v[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) v[j] = raw2(c0 + j * kStride);
#pragma unroll
    for (int j = 0; j < kBatch; ++j) pin(v[j]);
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      v[j] = mask2(c0 + j * kStride, v[j]);
      s0 = fmaf(v[j].x, v[j].x, s0);
      s1 = fmaf(v[j].y, v[j].y, s1);
    }
  }
  // rows of the wave that hold the same positions: lanes prow + k * kLPR
#pragma unroll
  for (int m = kLPR; m < 64; m <<= 1) {
    s0 += __shfl_xor(s0, m, 64);
    s1 += __shfl_xor(s1, m, 64);
  }
  if (crow == 0) {
    s_ss[wave][kPL * prow] = s0;
    if constexpr (kPL == 2) s_ss[wave][kPL * prow + 1] = s1;
  }
  __syncthreads();
  float q0 = 0.f, q1 = 0.f;
#pragma unroll
  for (int i = 0; i < kNormWaves; ++i) {
    q0 += s_ss[i][kPL * prow];
    if constexpr (kPL == 2) q1 += s_ss[i][kPL * prow + 1];
  }
  const float r0 = rsqrtf(q0 / (float)C + eps);
  const float r1 = rsqrtf(q1 / (float)C + eps);
  auto put = [&](int c, float2 v, float gw) {
    T* p = ob + (size_t)c * L + t;
    if constexpr (kPL == 1) {
      if (ok0) Elem<T>::store1(p, v.x * r0 * gw);
    } else if constexpr (kPair) {
      if (ok0) Pair<T>::store(p, v.x * r0 * gw, v.y * r1 * gw);
    } else {
      if (ok0) Elem<T>::store1(p, v.x * r0 * gw);
      if (ok1) Elem<T>::store1(p + 1, v.y * r1 * gw);
    }
  };
#pragma unroll
  for (int i = 0; i < kHold; ++i) {
    const int c = c_first + i * kStride;
    if (c < C) put(c, held[i], gw_held[i]);
  }
  for (int c0 = c_first + kHold * kStride; c0 < C; c0 += kBatch * kStride) {
    float2 v[kBatch];
    float gw[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      v[j] = raw2(c0 + j * kStride);
      gw[j] = scale_of(c0 + j * kStride);
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j)
      if (c0 + j * kStride < C) put(c0 + j * kStride, v[j], gw[j]);
  }
}

template <typename T, int kPos, int kPL, bool kPair>
hipError_t launch_norm_shape(const T* x, const T* w, float eps, T* out, int B, int C, int L,
                             hipStream_t st) {
  constexpr int kLine = 128 / (int)sizeof(T);  // elements per 128-byte line
  constexpr int kShare = kPos >= kLine ? 1 : kLine / kPos;
  const int tiles_per_row = (L + kPos - 1) / kPos;
  const int ntiles = B * tiles_per_row;
  const int unit = kNormXcds * kShare;
  const dim3 grid((unsigned)((ntiles + unit - 1) / unit * unit));
  hipLaunchKernelGGL((rms_norm_cm_kernel<T, kPos, kPL, kPair, kShare>), grid, dim3(kNormThreads),
                     0, st, x, w, eps, out, C, L, tiles_per_row, ntiles);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_norm_t(const void* x, const void* w, float eps, void* out, int B, int C, int L,
                         bool pair, hipStream_t st) {
  ProfScope prof("rms_norm_cm", st);
  auto* xp = static_cast<const T*>(x);
  auto* wp = static_cast<const T*>(w);
  auto* op = static_cast<T*>(out);
  // shapes from a sweep on MI355X at (4, 1024, 2048): 32 positions x 2 per
  // lane took 9.2 us (bf16) against 20 us for 128-position tiles
  if (pair) return launch_norm_shape<T, 32, 2, true>(xp, wp, eps, op, B, C, L, st);
  return launch_norm_shape<T, 16, 1, false>(xp, wp, eps, op, B, C, L, st);
}

}  // namespace

hipError_t launch_rms_norm_cm(int bf16, const void* x, const void* w, float eps, void* out, int B,
                              int C, int L, bool pair, hipStream_t st) {
  return bf16 ? launch_norm_t<__hip_bfloat16>(x, w, eps, out, B, C, L, pair, st)
              : launch_norm_t<float>(x, w, eps, out, B, C, L, pair, st);
}

}  // namespace ssm
