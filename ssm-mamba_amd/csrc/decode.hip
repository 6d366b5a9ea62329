// Fused decode step of the Mamba block for gfx950: the per-token work of
// Block.step / Mamba.step (modules/block.py:80-86, modules/mamba.py:189-243 of
// the reference) as four kernels per layer instead of a score of torch ops:
//
//   gemv_kernel (norm, conv epilogue)  xz = W_in @ rmsnorm(x); for the x half
//                                      xc = silu(window . w + xs w_last + b),
//                                      window roll
//   gemv_kernel                        p = W_x @ xc                    (B, R+2N)
//   ssm_step_kernel                    delta = W_dt @ p[:R];
//                                      state update with B = p[R:R+N],
//                                      C = p[R+N:]; y = (C.h + D*xc) * silu(z)
//   gemv_kernel (residual)             x' = x + W_out @ y
//
// or in three, with p = W_x @ xc folded into the other two: each in-projection
// workgroup of the x half writes the fp32 partial W_x[:, its channels] @ xc,
// and every ssm_step workgroup adds the partials of its batch row in a fixed
// order (kEpiConvX / kParts below); or, for a whole stack of layers, in one
// persistent launch that runs those three kernels' workgroups as phases, the
// workgroups handing activations to each other through flagged 8-byte units
// instead of grid barriers (decode_layers_kernel).
//
// and the LM head as gemv_kernel with the final norm.  Batch is small (one
// token per sequence), so every kernel is a weight stream: a wave owns a few
// weight rows, each lane issues all of its 16-byte row loads before any
// arithmetic, the workgroup stages the (tiny) activation rows in LDS meanwhile,
// and every weight chunk is applied to all batch rows.  Activations, weights and norm/conv/dt
// parameters share the element type T; accumulation is fp32; the SSM state
// stays fp32.
#include "ss_common.cuh"
#include "ss_io.cuh"
#include "ss_prof.h"

namespace ssm {

namespace {

constexpr int kDecThreads = 256;
constexpr int kGemvPass = 4;     // 16-byte chunks per lane per row per pass
constexpr int kMaxDecBatch = 8;  // batch rows per launch

template <typename T>
struct Chunk;  // 16 bytes of T

template <>
struct Chunk<float> {
  static constexpr int E = 4;
  using Raw = float4;
  __device__ static __forceinline__ void cvt(const Raw& r, float* v) {
    v[0] = r.x; v[1] = r.y; v[2] = r.z; v[3] = r.w;
  }
  __device__ static __forceinline__ Raw zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }
};

template <>
struct Chunk<__hip_bfloat16> {
  static constexpr int E = 8;
  using Raw = uint4;
  __device__ static __forceinline__ void cvt(const Raw& r, float* v) {
    v[0] = bf16_lo(r.x); v[1] = bf16_hi(r.x); v[2] = bf16_lo(r.y); v[3] = bf16_hi(r.y);
    v[4] = bf16_lo(r.z); v[5] = bf16_hi(r.z); v[6] = bf16_lo(r.w); v[7] = bf16_hi(r.w);
  }
  __device__ static __forceinline__ Raw zero() { return make_uint4(0u, 0u, 0u, 0u); }
};

template <typename T>
__device__ __forceinline__ typename Chunk<T>::Raw ldchunk(const T* __restrict__ p) {
  return *reinterpret_cast<const typename Chunk<T>::Raw*>(p);
}
// The same with a nontemporal load: the GEMV weights, read once per call and
// (a whole model's worth per token step) far more than the caches hold.
// Measured at config 4: the layer chain 686 -> 681 us, the step 0.738 ->
// 0.732 ms, the same bits.
template <typename T>
__device__ __forceinline__ typename Chunk<T>::Raw ldchunk_nt(const T* __restrict__ p) {
  typedef unsigned v4 __attribute__((ext_vector_type(4)));
  const v4 x = __builtin_nontemporal_load(reinterpret_cast<const v4*>(p));
  typename Chunk<T>::Raw r;
  __builtin_memcpy(&r, &x, 16);
  return r;
}

// Totals over the wave of NV per-lane values: afterwards out[g] of lane l is
// the sum over all lanes of v[g * 16 + (l >> 2)] (zero past NV); the four
// lanes of a quad agree.  permlane/DPP reduce-scatter, no LDS round trips.
template <int NV>
__device__ __forceinline__ void wave_totals(const float (&v)[NV], float (&out)[(NV + 15) / 16],
                                            int lane) {
#pragma unroll
  for (int g = 0; g < (NV + 15) / 16; ++g) {
    float t[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) t[i] = g * 16 + i < NV ? v[g * 16 + i] : 0.0f;
    wave_reduce16(t, lane);
    out[g] = t[0];
  }
}

// value rounded to T and back (the reference keeps these intermediates as T tensors)
template <typename T>
__device__ __forceinline__ float round_to(float v) {
  T t;
  Elem<T>::store1(&t, v);
  return Elem<T>::load1(&t);
}

// ---------------------------------------------------------------------------
// Device-scope accesses.  The workgroups of the layer-chain kernel (below) hand
// activations to each other inside one launch.  gfx950 has one L2 per XCD and
// the L2s are not coherent with each other, so such data is stored with SC1
// (written through to memory: device scope) and loaded with SC1 (not served
// from a possibly stale L2 line).  Buffer accesses carry the cache policy; the
// descriptors span whole tensors, so the range check drops nothing.
constexpr int kSC1 = 16;  // cache-policy bit SC1 of a buffer access

__device__ __forceinline__ __amdgpu_buffer_rsrc_t dev_rsrc(const void* base, size_t bytes) {
  return raw_rsrc(const_cast<void*>(base), (uint32_t)bytes);
}

// LL units ("low latency", as in RCCL's protocol of that name): 8 bytes of
// {data word, flag word}, written with one 8-byte store (single-copy atomic)
// and read with 8- or 16-byte loads, each 8-byte half again atomic, all at
// device scope.  A consumer polls the units it needs until every flag equals
// the launch's flag: the data arrive with their own readiness, in one memory
// round trip, with no barrier and no separate flag.
__device__ __forceinline__ void ll_put(__amdgpu_buffer_rsrc_t r, uint32_t unit, uint32_t data,
                                       uint32_t flag) {
  const u32x2_v v = {data, flag};
  __builtin_amdgcn_raw_buffer_store_b64(v, r, (int)(unit * 8u), 0, kSC1);
}
// units unit and unit + 1: {data0, flag0, data1, flag1}
__device__ __forceinline__ u32x4_v ll_get2(__amdgpu_buffer_rsrc_t r, uint32_t unit) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)(unit * 8u), 0, kSC1);
}
__device__ __forceinline__ u32x2_v ll_get1(__amdgpu_buffer_rsrc_t r, uint32_t unit) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, (int)(unit * 8u), 0, kSC1);
}

__device__ __forceinline__ unsigned dev_load_u32(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void dev_store_u32(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned dev_add_u32(unsigned* p, unsigned v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Bounded wait on LL units: pairs[i] (units pairs[i], pairs[i] + 1) of the
// lanes with need set.  Re-reads only the pairs not yet ready.  false after
// maxspin polls or once the error word is set (some other workgroup gave up).
struct LLWait {
  unsigned flag, maxspin;
  const unsigned* err;
};

template <int N>
__device__ __forceinline__ bool ll_wait2(__amdgpu_buffer_rsrc_t r, const uint32_t (&pairs)[N],
                                         bool need, const LLWait& w, u32x4_v (&v)[N]) {
  if (!need) return true;
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = ll_get2(r, pairs[i]);
  for (unsigned n = 0;; ++n) {
    bool ready = true;
#pragma unroll
    for (int i = 0; i < N; ++i) ready &= (v[i][1] == w.flag) & (v[i][3] == w.flag);
    if (ready) return true;
    if (n >= w.maxspin || ((n & 63) == 63 && dev_load_u32(w.err) != 0)) return false;
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int i = 0; i < N; ++i)
      if ((v[i][1] != w.flag) | (v[i][3] != w.flag)) v[i] = ll_get2(r, pairs[i]);
  }
}

__device__ __forceinline__ bool ll_wait1(__amdgpu_buffer_rsrc_t r, uint32_t unit, const LLWait& w,
                                         u32x2_v& v) {
  v = ll_get1(r, unit);
  for (unsigned n = 0; v[1] != w.flag; ++n) {
    if (n >= w.maxspin || ((n & 63) == 63 && dev_load_u32(w.err) != 0)) return false;
    __builtin_amdgcn_s_sleep(1);
    v = ll_get1(r, unit);
  }
  return true;
}

// the data word of an LL unit as values of T: two bf16 (low half first) or one fp32
template <typename T> struct LLVal;
template <> struct LLVal<__hip_bfloat16> {
  static constexpr int V = 2;
  __device__ static __forceinline__ float get(uint32_t w, int i) { return i ? bf16_hi(w) : bf16_lo(w); }
  __device__ static __forceinline__ uint32_t pack(float a, float b) { return pack_bf16x2(a, b); }
};
template <> struct LLVal<float> {
  static constexpr int V = 1;
  __device__ static __forceinline__ float get(uint32_t w, int) { return __uint_as_float(w); }
  __device__ static __forceinline__ uint32_t pack(float a, float) { return __float_as_uint(a); }
};

enum GemvEpi { kEpiPlain = 0, kEpiConv = 1, kEpiConvX = 2 };

// x-projection partials: the in-projection with them runs kXRows weight rows
// per wave, so each workgroup covers kXBlock channels of the x half
constexpr int kXRows = 4;
constexpr int kXBlock = (kDecThreads / 64) * kXRows;
constexpr int kMaxXOut = 256;    // R + 2N limit of the folded x-projection
constexpr int kPartLoads = 16;   // partial float4 loads in flight per thread

struct GemvArgs {
  const void* W;     // (O, K)
  const void* x;     // (B, K)
  const void* nw;    // (K) RMSNorm weight (kNorm)
  float eps;
  const void* bias;  // (O) nullable
  const void* res;   // (B, O) nullable (plain epilogue)
  void* y;           // (B, O)
  int B, O, K;
  // conv epilogue: rows o < dim are xs; window (B, dim, width-1), weight (dim, width)
  int dim, width;
  void* ctx;
  const void* cw;
  const void* cb;    // nullable
  void* xc;          // (B, dim)
  // kEpiConvX: part (dim / kXBlock, B, nout4) fp32 = W_x (nout, dim) partials
  const void* Wx;
  int nout, nout4;
  float* part;       // (the layer chain: LL units, flag below)
  unsigned flag;
};

// One workgroup's share of y[b, o] = scale_b * sum_k W[o, k] * (1 + nw[k])^[kNorm] * x[b, k]
// (+ bias[o]) (+ res[b, o]), scale_b = rsqrt(mean_k x[b, k]^2 + eps) with kNorm,
// else 1 -- i.e. W @ rmsnorm(x).
//
// The workgroup has kWaves waves: kWaves / kKSplit row waves of kRows rows
// each, times kKSplit K-slices.  Per pass of PK = kKSplit * kPass * 64 * E
// columns, the wave of slice s holds kPass 16-byte chunks per row of the
// columns [s kPass 64 E, (s+1) kPass 64 E) of the pass; each lane issues all
// of its weight loads (load_pass), then the workgroup stages x[:, pass] in LDS
// (and accumulates x^2 for the norm), then the weights meet the staged
// activations (run_pass).  With K-slices the waves' totals of a row are added
// in slice order through LDS.  kEpiConv adds the Mamba conv step for the x half
// of the in-projection (rows o < dim): xc = silu(window . w + xs w + cb), and
// the window rolls by one.  kEpiConvX also writes this workgroup's x-projection
// partial part[blk, b, j] = sum_{c in blk} W_x[j, c] xc[b, c].
//
// The steps are separate so that the layer-chain kernel can issue a phase's
// weight and operand loads before it waits for the phase's input.  kChain
// (the layer chain): x arrives as LL units (stage_ll) or from the launch's
// input, the residual comes from LL units (res_ll) or the launch's input, and
// the results go to the workgroup's LDS tile (yt, and xc for the x half) and,
// for the x-projection partials, to LL units; the caller packs the tile into
// LL units.  The conv window is private to the workgroup that owns its
// channels and is accessed directly either way.
template <typename T, int kMB, int kRows, bool kNorm, int kEpi, int kWaves = 4, int kKSplit = 1,
          int kPass = kGemvPass, int kTaps = 8>
struct GemvWork {
  static constexpr int E = Chunk<T>::E;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kRowWaves = kWaves / kKSplit;
  static constexpr bool kXP = kEpi == kEpiConvX;
  static constexpr int kXB = kRowWaves * kRows;      // rows (channels) per workgroup
  static_assert(!kXP || kXB == kXBlock, "x-projection partials cover kXBlock channels per workgroup");
  static_assert(kRowWaves * kKSplit == kWaves, "waves split evenly into K-slices");
  static constexpr int kXC = kXP ? kXBlock / E : 1;  // 16-byte chunks of one W_x row slice
  static constexpr int span = 64 * E;                // columns of one chunk step of a wave
  static constexpr int kSliceCols = kPass * span;    // columns of one K-slice per pass
  static constexpr int PK = kKSplit * kSliceCols;    // columns per pass
  static constexpr int kStage = PK / E;              // staged chunks per batch row and pass
  static_assert(kStage % 64 == 0 && kStage <= kThreads, "one staged chunk per thread of whole waves");
  static constexpr int kStageWaves = kStage / 64;
  static constexpr int kNV = kRows * kMB;
  static constexpr int kNG = (kNV + 15) / 16;
  static constexpr int kMaxTaps = kTaps;  // conv width limit (kEpiConv*)
  using Raw = typename Chunk<T>::Raw;

  // LDS of one workgroup
  struct Smem {
    __align__(16) T sx[kMB][PK];                       // staged activations of a pass
    float red[kWaves][kMB];                            // per-wave sums of x^2
    float scale[kMB];                                  // RMSNorm scale per batch row
    float xc[kXP ? kMB : 1][kXP ? kXBlock : 1];        // conv outputs of the block
    float kst[kKSplit > 1 ? kKSplit - 1 : 1][kRowWaves][kNV];  // totals of slices 1..
    float yt[kMB][kXB];                                // results of the block (kChain)
  };

  int lane, wave, ks, row0, xblk0;
  // epilogue operands of this lane's outputs (group g: output i = g * 16 + (lane >> 2),
  // i = r * kMB + b)
  int e_row[kNG], e_b[kNG];
  bool e_ok[kNG];
  float e_bias[kNG], e_res[kNG], e_cb[kNG];
  float e_cw[kNG][kMaxTaps], e_win[kNG][kMaxTaps - 1];
  Raw xw[kXC];                        // the W_x slice of output j = threadIdx.x
  Raw wr[kRows][kPass];               // weights of the current pass
  float xs_keep[kNG];                 // kChain conv epilogue: the window's new last column
  Raw nwr[kNorm ? kPass : 1];         // norm weights of the current pass
  float acc[kRows][kMB];
  float ssq[kMB];

  __device__ __forceinline__ void begin(int blk) {
    lane = threadIdx.x & 63;
    wave = threadIdx.x >> 6;
    ks = wave / kRowWaves;
    row0 = (blk * kRowWaves + wave % kRowWaves) * kRows;
    xblk0 = blk * kXB;
#pragma unroll
    for (int b = 0; b < kMB; ++b) {
      ssq[b] = 0.0f;
#pragma unroll
      for (int r = 0; r < kRows; ++r) acc[r][b] = 0.0f;
    }
  }

  // Epilogue operands (bias, residual, conv taps and window) of this lane's
  // outputs and the W_x slice, fetched before the weight stream so their
  // latency overlaps it.  Every lane loads, from clamped addresses (absent
  // operands from a valid stand-in), so no load sits in a branch: a load inside
  // a branch is waited for inside it, which would serialise these round trips.
  // kChain: the residual comes from the LL units res_ll when given (their
  // flags are not checked: this workgroup has already waited for all of them),
  // else from res, which a kernel before the launch wrote.
  template <bool kChain>
  __device__ __forceinline__ void load_epilogue(const GemvArgs& a, Smem& sm, const void* res_ll = nullptr) {
    const T* __restrict__ W = static_cast<const T*>(a.W);
    const int B = a.B, O = a.O;
#pragma unroll
    for (int g = 0; g < kNG; ++g) {
      const int i = g * 16 + (lane >> 2);
      const int rl = i / kMB;
      e_row[g] = row0 + rl;
      e_b[g] = i - rl * kMB;
      e_ok[g] = ks == 0 && (lane & 3) == 0 && i < kNV && e_row[g] < O && e_b[g] < B;
      const int rc = min(e_row[g], O - 1), bc = min(e_b[g], B - 1);
      e_bias[g] = Elem<T>::load1((a.bias ? static_cast<const T*>(a.bias) : W) + rc);
      e_res[g] = 0.0f;
      e_cb[g] = 0.0f;
#pragma unroll
      for (int j = 0; j < kMaxTaps; ++j) e_cw[g][j] = 0.0f;
#pragma unroll
      for (int j = 0; j < kMaxTaps - 1; ++j) e_win[g][j] = 0.0f;
      if constexpr (kEpi == kEpiPlain) {
        if constexpr (kChain) {
          if (res_ll) {
            constexpr int V = LLVal<T>::V;
            const uint32_t i = (uint32_t)(bc * O + rc);
            const u32x2_v u = ll_get1(dev_rsrc(res_ll, (size_t)B * O / V * 8), i / V);
            e_res[g] = LLVal<T>::get(u[0], i % V);
          } else {
            e_res[g] = Elem<T>::load1(static_cast<const T*>(a.res) + (size_t)bc * O + rc);
          }
        } else {
          e_res[g] = Elem<T>::load1(a.res ? static_cast<const T*>(a.res) + (size_t)bc * O + rc : W + rc);
        }
      } else {
        const int wd = a.width;
        const int rx = min(rc, a.dim - 1);  // x-half row (rows past dim use none of these)
        const T* __restrict__ cw = static_cast<const T*>(a.cw) + (size_t)rx * wd;
        const T* __restrict__ win =
            static_cast<const T*>(a.ctx) + ((size_t)bc * a.dim + rx) * (wd - 1);
#pragma unroll
        for (int j = 0; j < kMaxTaps; ++j) e_cw[g][j] = Elem<T>::load1(cw + min(j, wd - 1));
#pragma unroll
        for (int j = 0; j < kMaxTaps - 1; ++j) e_win[g][j] = Elem<T>::load1(win + min(j, wd - 2));
        e_cb[g] = Elem<T>::load1(a.cb ? static_cast<const T*>(a.cb) + rx : cw);
      }
    }
    // the W_x slice of output j = threadIdx.x, ahead of the weight stream; xc
    // slots of rows this workgroup does not finish stay zero
#pragma unroll
    for (int c = 0; c < kXC; ++c) xw[c] = Chunk<T>::zero();
    if constexpr (kXP) {
      if (threadIdx.x < kMB * kXBlock) sm.xc[threadIdx.x / kXBlock][threadIdx.x % kXBlock] = 0.0f;
      // clamped row and block (dim >= kXBlock); rows past nout are zeroed at use
      const int jr = min((int)threadIdx.x, a.nout - 1);
      const T* __restrict__ wx =
          static_cast<const T*>(a.Wx) + (size_t)jr * a.dim + min(xblk0, a.dim - kXBlock);
#pragma unroll
      for (int c = 0; c < kXC; ++c) xw[c] = ldchunk(wx + c * E);
    }
  }

  // this lane's weight chunks of the pass at column kb (and the norm weight
  // of its columns, clamped past K where the chunk is not used)
  // After finish<true> with the conv epilogue: the conv window roll (drop the
  // oldest column, append x).  The layer chain calls it after the phase's
  // hand-off stores, which the other workgroups wait for; the window is read
  // again only at the next token step.
  __device__ __forceinline__ void store_window(const GemvArgs& a) {
    if constexpr (kEpi != kEpiPlain) {
#pragma unroll
      for (int g = 0; g < kNG; ++g) {
        if (!e_ok[g] || e_row[g] >= a.dim) continue;
        const int wd = a.width;
        T* __restrict__ win = static_cast<T*>(a.ctx) + ((size_t)e_b[g] * a.dim + e_row[g]) * (wd - 1);
#pragma unroll
        for (int j = 0; j + 1 < kMaxTaps - 1; ++j)
          if (j + 1 < wd - 1) Elem<T>::store1(win + j, e_win[g][j + 1]);
        Elem<T>::store1(win + wd - 2, xs_keep[g]);
      }
    }
  }

  __device__ __forceinline__ void load_pass(const GemvArgs& a, int kb) {
    const T* __restrict__ W = static_cast<const T*>(a.W);
    const int O = a.O, K = a.K;
    const int k0 = kb + ks * kSliceCols;
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      const int row = min(row0 + r, O - 1);
#pragma unroll
      for (int c = 0; c < kPass; ++c) {
        if (k0 + c * span < K) {  // wave-uniform: whole chunks past K are not loaded
          const int kc = min(k0 + c * span + lane * E, K - E);
          wr[r][c] = ldchunk_nt(W + (size_t)row * K + kc);
        } else {
          wr[r][c] = Chunk<T>::zero();
        }
      }
    }
    if constexpr (kNorm) {
      const T* __restrict__ nw = static_cast<const T*>(a.nw);
#pragma unroll
      for (int c = 0; c < kPass; ++c) nwr[c] = ldchunk(nw + min(k0 + c * span + lane * E, K - E));
    }
  }

  // stage x[:, kb:kb+PK] (thread t < kStage owns chunk t of every batch row),
  // then accumulate the pass.  Loads from clamped addresses, zeroed past K by
  // a select (no load in a branch); slots of rows b >= B hold row B-1 and are
  // never read.
  __device__ __forceinline__ void run_pass(const GemvArgs& a, int kb, Smem& sm) {
    stage(a, kb, sm);
    accumulate(a, kb, sm);
  }

  // chunk v of batch row b into LDS, with its squares for the norm
  __device__ __forceinline__ void put_chunk(int b, Raw v, int B, Smem& sm) {
    *reinterpret_cast<Raw*>(&sm.sx[b][threadIdx.x * E]) = v;
    if constexpr (kNorm) {
      if (b < B) {
        float f[E];
        Chunk<T>::cvt(v, f);
#pragma unroll
        for (int i = 0; i < E; ++i) ssq[b] = fmaf(f[i], f[i], ssq[b]);
      }
    }
  }

  __device__ __forceinline__ void stage(const GemvArgs& a, int kb, Smem& sm) {
    const T* __restrict__ x = static_cast<const T*>(a.x);
    const int B = a.B, K = a.K;
    if (kStage == kThreads || (int)threadIdx.x < kStage) {
      const int k = kb + threadIdx.x * E;
      const int kc = min(k, K - E);
      Raw xr[kMB];
#pragma unroll
      for (int b = 0; b < kMB; ++b) xr[b] = ldchunk(x + (size_t)min(b, B - 1) * K + kc);
#pragma unroll
      for (int b = 0; b < kMB; ++b) {
        Raw v = xr[b];
        if (k >= K) v = Chunk<T>::zero();
        put_chunk(b, v, B, sm);
      }
    }
  }

  // stage x[:, 0:K] (one pass) from LL units x_ll (B, K / V units); false if
  // the wait gave up.  Chunk t of row b is the 4 units from (b K + t E) / V.
  __device__ __forceinline__ bool stage_ll(const GemvArgs& a, const void* x_ll, const LLWait& w,
                                           Smem& sm) {
    constexpr int V = LLVal<T>::V;
    static_assert(E / V == 4, "a 16-byte chunk is 4 LL units");
    const int B = a.B, K = a.K;
    const int k = threadIdx.x * E;
    const bool mine = (kStage == kThreads || (int)threadIdx.x < kStage) && k < K;
    const auto r = dev_rsrc(x_ll, (size_t)B * K / V * 8);
    uint32_t pairs[2 * kMB];
#pragma unroll
    for (int b = 0; b < kMB; ++b) {
      const uint32_t u0 = (uint32_t)((min(b, B - 1) * K + k) / V);
      pairs[2 * b] = u0;
      pairs[2 * b + 1] = u0 + 2;
    }
    u32x4_v v[2 * kMB];
    const bool ok = ll_wait2<2 * kMB>(r, pairs, mine, w, v);
    if (kStage == kThreads || (int)threadIdx.x < kStage) {
#pragma unroll
      for (int b = 0; b < kMB; ++b) {
        Raw c = Chunk<T>::zero();
        if (mine) {
          const uint32_t d[4] = {v[2 * b][0], v[2 * b][2], v[2 * b + 1][0], v[2 * b + 1][2]};
          c = *reinterpret_cast<const Raw*>(d);
        }
        put_chunk(b, c, B, sm);
      }
    }
    return ok;
  }

  __device__ __forceinline__ void accumulate(const GemvArgs& a, int kb, Smem& sm) {
    const int B = a.B, K = a.K;
    __syncthreads();
#pragma unroll
    for (int c = 0; c < kPass; ++c) {
      const int kl = ks * kSliceCols + c * span + lane * E;
      if (kb + kl < K) {
        float wf[kRows][E];
#pragma unroll
        for (int r = 0; r < kRows; ++r) Chunk<T>::cvt(wr[r][c], wf[r]);
        if constexpr (kNorm) {
          float nv[E];
          Chunk<T>::cvt(nwr[c], nv);
#pragma unroll
          for (int r = 0; r < kRows; ++r)
#pragma unroll
            for (int i = 0; i < E; ++i) wf[r][i] *= 1.0f + nv[i];
        }
        // every batch row's activations first (rows past B repeat row B - 1,
        // whose sums are never used): no branch per row, so the LDS reads are
        // all in flight together instead of one round trip per row
        Raw xr[kMB];
#pragma unroll
        for (int b = 0; b < kMB; ++b) xr[b] = *reinterpret_cast<const Raw*>(&sm.sx[min(b, B - 1)][kl]);
#pragma unroll
        for (int b = 0; b < kMB; ++b) {
          float v[E];
          Chunk<T>::cvt(xr[b], v);
#pragma unroll
          for (int r = 0; r < kRows; ++r) {
            float s = acc[r][b];
#pragma unroll
            for (int i = 0; i < E; ++i) s = fmaf(wf[r][i], v[i], s);
            acc[r][b] = s;
          }
        }
      }
    }
    __syncthreads();
  }

  // norm scale, wave totals (and the slices' sum) and the epilogue
  template <bool kChain>
  __device__ __forceinline__ void finish(const GemvArgs& a, Smem& sm) {
    const int B = a.B, O = a.O, K = a.K;
    if constexpr (kNorm) {
      // only the staging waves hold sums of squares
      float st[(kMB + 15) / 16];
      wave_totals<kMB>(ssq, st, lane);
      if (wave < kStageWaves && (lane & 3) == 0 && (lane >> 2) < kMB) sm.red[wave][lane >> 2] = st[0];
      __syncthreads();
      if (threadIdx.x < kMB) {
        const int b = threadIdx.x;
        float t = sm.red[0][b];
#pragma unroll
        for (int w = 1; w < kStageWaves; ++w) t += sm.red[w][b];
        sm.scale[b] = rsqrtf(t / (float)K + a.eps);
      }
      __syncthreads();
    }
    // the W_x slice as floats now, while its (oldest) loads are known complete:
    // converted after the epilogue's stores, it would wait for those too
    float xwf[kXP ? kXBlock : 1];
    if constexpr (kXP) {
#pragma unroll
      for (int c = 0; c < kXC; ++c) Chunk<T>::cvt(xw[c], xwf + c * E);
      if ((int)threadIdx.x >= a.nout) {  // padding columns of the partial
#pragma unroll
        for (int c = 0; c < kXBlock; ++c) xwf[c] = 0.0f;
      }
      // keep the conversion here (the compiler would sink it to its use)
#pragma unroll
      for (int c = 0; c < kXBlock; ++c) asm volatile("" : "+v"(xwf[c]));
    }
    // wave totals: lane 4i (+0..3) of group g finishes output i = g * 16 + (lane >> 2)
    float tot[kNG];
    {
      float flat[kNV];
#pragma unroll
      for (int r = 0; r < kRows; ++r)
#pragma unroll
        for (int b = 0; b < kMB; ++b) flat[r * kMB + b] = acc[r][b];
      wave_totals<kNV>(flat, tot, lane);
    }
    if constexpr (kKSplit > 1) {
      // slices 1.. hand their totals to slice 0, which adds them in slice order
      const int rw = wave % kRowWaves;
      if (ks > 0) {
#pragma unroll
        for (int g = 0; g < kNG; ++g) {
          const int i = g * 16 + (lane >> 2);
          if ((lane & 3) == 0 && i < kNV) sm.kst[ks - 1][rw][i] = tot[g];
        }
      }
      __syncthreads();
      if (ks == 0) {
#pragma unroll
        for (int g = 0; g < kNG; ++g) {
          const int i = min(g * 16 + (lane >> 2), kNV - 1);
#pragma unroll
          for (int s = 0; s < kKSplit - 1; ++s) tot[g] += sm.kst[s][rw][i];
        }
      }
    }
    T* __restrict__ y = static_cast<T*>(a.y);
#pragma unroll
    for (int g = 0; g < kNG; ++g) {
      if (!e_ok[g]) continue;
      const int row = e_row[g], bl = e_b[g];
      float s = tot[g];
      if constexpr (kNorm) s *= sm.scale[bl];
      if (a.bias) s += e_bias[g];
      if constexpr (kEpi == kEpiPlain) {
        const float v = (kChain || a.res) ? s + e_res[g] : s;
        if constexpr (kChain) sm.yt[bl][row - xblk0] = v;
        else Elem<T>::store1(y + (size_t)bl * O + row, v);
      } else {
        if constexpr (kChain) sm.yt[bl][row - xblk0] = s;
        else Elem<T>::store1(y + (size_t)bl * O + row, s);
        if (row < a.dim) {
          const int wd = a.width;
          const float xs = round_to<T>(s);
          float cv = a.cb ? e_cb[g] : 0.0f;
          float wlast = 0.0f;
#pragma unroll
          for (int j = 0; j < kMaxTaps; ++j) {
            if (j < wd - 1) cv = fmaf(e_cw[g][j], e_win[g][j], cv);
            if (j == wd - 1) wlast = e_cw[g][j];
          }
          cv = fmaf(wlast, xs, cv);
          const float xcv = round_to<T>(silu_f(cv));
          if constexpr (!kChain) Elem<T>::store1(static_cast<T*>(a.xc) + (size_t)bl * a.dim + row, xcv);
          if constexpr (kXP) sm.xc[bl][row - xblk0] = xcv;
          if constexpr (kChain) {
            xs_keep[g] = xs;  // see store_window
          } else {
            T* __restrict__ win = static_cast<T*>(a.ctx) + ((size_t)bl * a.dim + row) * (wd - 1);
#pragma unroll
            for (int j = 0; j + 1 < kMaxTaps - 1; ++j)
              if (j + 1 < wd - 1) Elem<T>::store1(win + j, e_win[g][j + 1]);
            Elem<T>::store1(win + wd - 2, xs);
          }
        }
      }
    }
    if constexpr (kXP) {
      __syncthreads();
      if (xblk0 < a.dim && (int)threadIdx.x < a.nout4) {
        const int blk = xblk0 / kXBlock;
        const size_t p0 = (size_t)blk * B * a.nout4 + threadIdx.x;
        const auto prs = dev_rsrc(a.part, (size_t)(a.dim / kXBlock) * B * a.nout4 * 8);
        // all rows' sums first (rows past B repeat row B - 1), then the stores
        float ps[kMB];
#pragma unroll
        for (int b = 0; b < kMB; ++b) {
          const int bc = min(b, B - 1);
          float s = 0.0f;
#pragma unroll
          for (int c = 0; c < kXBlock; ++c) s = fmaf(xwf[c], sm.xc[bc][c], s);
          ps[b] = s;
        }
#pragma unroll
        for (int b = 0; b < kMB; ++b) {
          if (b < B) {
            if constexpr (kChain) ll_put(prs, (uint32_t)(p0 + (size_t)b * a.nout4), __float_as_uint(ps[b]), a.flag);
            else a.part[p0 + (size_t)b * a.nout4] = ps[b];
          }
        }
      }
    }
  }
};

template <typename T, int kMB, int kRows, bool kNorm, int kEpi>
__global__ __launch_bounds__(kDecThreads) void gemv_kernel(const GemvArgs a) {
  using Work = GemvWork<T, kMB, kRows, kNorm, kEpi>;
  __shared__ typename Work::Smem sm;
  Work w;
  w.begin(blockIdx.x);
  w.template load_epilogue<false>(a, sm);
  for (int kb = 0; kb < a.K; kb += Work::PK) {
    w.load_pass(a, kb);
    w.run_pass(a, kb, sm);
  }
  w.template finish<false>(a, sm);
}

struct SsmArgs {
  const void* pp;    // params (B, nout), or the fp32 partials (nparts, B, nout4)
  int nout, nout4, nparts, R;
  const void* Wdt;   // (dim, R)
  const void* dt_bias;
  const void* logA;  // (dim, N)
  const void* Dv;
  const void* xc;    // (B, dim)
  const void* xz;    // (B, ld_xz): z = xz[:, dim:2*dim]
  int ld_xz;
  float* state;      // (B, dim, N) fp32
  void* y;           // (B, dim)
  int dim, B;
};

// Step-size projection, state update and gate, kSplit threads per (b, d), each
// with kN / kSplit of the states:
//   delta = round_T(W_dt[d, :R] . p[b, :R]); delta' = softplus(delta + dt_bias[d])
//   h' = exp(delta' A) h + delta' xc B,  A = -exp(log_A), B = p[b, R:R+N]
//   y = (sum_n C h' + D xc) * silu(z),   C = p[b, R+N:R+2N], z = xz[b, dim + d]
// (modules/mamba.py:216-240 with selective_update/kernel.cu:39-71; the T
// roundings mirror the reference's intermediate T tensors).  A workgroup of
// kThreads = kChan kSplit threads covers kChan channels of one batch row.  With
// kSplit > 1 the threads of a channel (adjacent lanes) split the dt dot
// product by chunks and the output sum by states, and combine both with
// butterfly adds (a fixed order).
//
// kParts: p is not given; pp holds the in-projection's fp32 x-projection
// partials (nparts, batch, nout4) and p[b] = round_T(sum over the partials),
// added in a fixed order: thread group s of S = kThreads / (nout4 / 4) sums
// partials [s nparts / S, (s+1) nparts / S) in turn, then the S group sums in
// turn.
//
// As with GemvWork, the loads come in separate steps (the partials, the
// operands that do not depend on p, and the activations xc and z).  The layer
// chain reads xc and z as LL units, sums the partials itself into s_p and
// calls compute<true>, which leaves y in an LDS tile and keeps the new state
// in registers until store_state.
template <typename T, int kN, bool kVecR, bool kParts, int kSplit = 1, int kPL = kPartLoads,
          int kMaxRC = 16, int kChan = kDecThreads>
struct SsmStep {
  static constexpr int E = Chunk<T>::E;
  static constexpr int kThreads = kChan * kSplit;
  static constexpr int kNS = kN / kSplit;               // states per thread
  static_assert((kNS % 4 == 0 || kNS == 2) && (kSplit & (kSplit - 1)) == 0,
                "whole float4 (or one float2) state groups per thread");
  static constexpr int kSV = kNS < 4 ? kNS : 4;  // states per vector load / store
  using SV = typename std::conditional<kSV == 4, float4, float2>::type;
  // dt-projection chunks per row: R <= kMaxRC E
  static constexpr int kRC = kMaxRC / kSplit;           // of them held by one thread
  using Raw = typename Chunk<T>::Raw;

  int b, d, dc, q, ng, S, sg, gi, w0, w1;
  float4 pv[kParts ? kPL : 1];
  Raw wv[kVecR ? kRC : 1];
  float hs[kNS];  // this thread's states
  float la[kNS];
  float bias_v, dv_v, u, z;
  u32x2_v act_u, act_z;  // the chain's xc and z units as first read

  __device__ __forceinline__ void begin(const SsmArgs& a, int dblk, int brow) {
    b = brow;
    q = threadIdx.x % kSplit;
    d = dblk * kChan + threadIdx.x / kSplit;
    dc = min(d, a.dim - 1);
    ng = a.nout4 >> 2;
    S = kParts ? kThreads / ng : 1;
    sg = threadIdx.x / ng;
    gi = threadIdx.x - sg * ng;
    w0 = sg * a.nparts / S;
    w1 = (sg + 1) * a.nparts / S;
  }

  // partial block w of this thread's float4 column
  __device__ __forceinline__ float4 part(const SsmArgs& a, int w) const {
    const size_t i = (size_t)b * ng + gi + (size_t)w * a.B * ng;
    return reinterpret_cast<const float4*>(a.pp)[i];
  }

  // partial loads first in the stand-alone kernel: they are the longest chain.
  // Clamped (always valid) partial indexes, unused ones skipped in the sum: no
  // load in a branch, so all of them are in flight at once.
  __device__ __forceinline__ void load_parts(const SsmArgs& a) {
    if constexpr (kParts) {
#pragma unroll
      for (int j = 0; j < kPL; ++j) pv[j] = part(a, min(w0 + j, a.nparts - 1));
    }
  }

  // this thread's operands that do not depend on p (dt-projection chunks
  // c = q + kSplit j, states [q kNS, (q+1) kNS))
  __device__ __forceinline__ void load_operands(const SsmArgs& a) {
    const T* __restrict__ Wdt = static_cast<const T*>(a.Wdt);
    const T* __restrict__ logA = static_cast<const T*>(a.logA);
    const T* __restrict__ wrow = Wdt + (size_t)dc * a.R;
    if constexpr (kVecR) {
#pragma unroll
      for (int j = 0; j < kRC; ++j) {
        const int c = q + kSplit * j;
        wv[j] = c * E < a.R ? ldchunk(wrow + c * E) : Chunk<T>::zero();
      }
    }
    const float* __restrict__ h = a.state + ((size_t)b * a.dim + dc) * kN + q * kNS;
#pragma unroll
    for (int g = 0; g < kNS / kSV; ++g) {
      const SV v = *reinterpret_cast<const SV*>(h + kSV * g);
      __builtin_memcpy(&hs[kSV * g], &v, sizeof(v));
    }
#pragma unroll
    for (int n = 0; n < kNS; ++n) la[n] = Elem<T>::load1(logA + (size_t)dc * kN + q * kNS + n);
    // absent dt_bias / D read a valid stand-in (log_A) and are dropped at use:
    // loads in a branch would be waited for there
    bias_v = Elem<T>::load1((a.dt_bias ? static_cast<const T*>(a.dt_bias) : logA) + dc);
    dv_v = Elem<T>::load1((a.Dv ? static_cast<const T*>(a.Dv) : logA) + dc);
  }

  __device__ __forceinline__ void load_act(const SsmArgs& a) {
    u = Elem<T>::load1(static_cast<const T*>(a.xc) + (size_t)b * a.dim + dc);
    z = Elem<T>::load1(static_cast<const T*>(a.xz) + (size_t)b * a.ld_xz + a.dim + dc);
  }

  // the layer chain: xc and z of this thread's channel from LL units (B, dim / V)
  // at a.xc and a.xz.  issue_act_ll reads both units once, ahead of the wait
  // for the partial sums: they are written in the in-projection phase, before
  // the partials' slice sums exist, so they are normally there, and their
  // round trip runs under that wait instead of after it.  load_act_ll then
  // polls again only for a unit whose flag was not yet set.
  __device__ __forceinline__ void issue_act_ll(const SsmArgs& a) {
    constexpr int V = LLVal<T>::V;
    const uint32_t i = (uint32_t)(b * a.dim + dc);
    const size_t bytes = (size_t)a.B * a.dim / V * 8;
    act_u = ll_get1(dev_rsrc(a.xc, bytes), i / V);
    act_z = ll_get1(dev_rsrc(a.xz, bytes), i / V);
  }
  __device__ __forceinline__ bool load_act_ll(const SsmArgs& a, const LLWait& w) {
    constexpr int V = LLVal<T>::V;
    const uint32_t i = (uint32_t)(b * a.dim + dc);
    const size_t bytes = (size_t)a.B * a.dim / V * 8;
    u32x2_v vu = act_u, vz = act_z;
    const bool ok_u = vu[1] == w.flag || ll_wait1(dev_rsrc(a.xc, bytes), i / V, w, vu);
    const bool ok_z = vz[1] == w.flag || ll_wait1(dev_rsrc(a.xz, bytes), i / V, w, vz);
    u = LLVal<T>::get(vu[0], i % V);
    z = LLVal<T>::get(vz[0], i % V);
    return ok_u && ok_z;
  }

  // sum of v over the kSplit adjacent lanes of a channel (butterfly).  Within
  // a quad the partners are DPP quad permutations (no LDS round trip, as a
  // shuffle would take); a + b = b + a, so every lane gets the same sum.
  __device__ __forceinline__ float split_sum(float v) const {
    if constexpr (kSplit >= 2) v += dpp_mov<kDppQuadXor1>(v);
    if constexpr (kSplit >= 4) v += dpp_mov<kDppQuadXor2>(v);
#pragma unroll
    for (int m = 4; m < kSplit; m <<= 1) v += __shfl_xor(v, m, 64);
    return v;
  }

  // s_p: [nout4] floats; s_red: [S][nout4 / 4] float4 (S * nout4 <= 4 kThreads)
  __device__ __forceinline__ void finish(const SsmArgs& a, float* s_p, float4* s_red) {
    const int nout = a.nout, nout4 = a.nout4;
    if constexpr (kParts) {
      float4 pacc = make_float4(0.f, 0.f, 0.f, 0.f);
      if (sg < S) {
        for (int wb = w0;; wb += kPL) {
#pragma unroll
          for (int j = 0; j < kPL; ++j) {
            if (wb + j < w1) {
              pacc.x += pv[j].x; pacc.y += pv[j].y; pacc.z += pv[j].z; pacc.w += pv[j].w;
            }
          }
          if (wb + kPL >= w1) break;
#pragma unroll
          for (int j = 0; j < kPL; ++j) pv[j] = part(a, min(wb + kPL + j, a.nparts - 1));
        }
        s_red[sg * ng + gi] = pacc;
      }
      __syncthreads();
      for (int i = threadIdx.x; i < nout; i += kThreads) {
        const float* r = reinterpret_cast<const float*>(s_red) + i;
        float t = 0.0f;
        for (int g = 0; g < S; ++g) t += r[g * nout4];
        s_p[i] = round_to<T>(t);
      }
    } else {
      const T* __restrict__ p = static_cast<const T*>(a.pp);
      for (int i = threadIdx.x; i < nout; i += kThreads) s_p[i] = Elem<T>::load1(p + (size_t)b * nout + i);
    }
    __syncthreads();
    compute<false>(a, s_p);
  }

  // delta, state update and gate from params s_p (in LDS, complete); s_y
  // (kChain): [256] floats, y of the workgroup's channels (0 past dim)
  template <bool kChain>
  __device__ __forceinline__ void compute(const SsmArgs& a, const float* s_p, float* s_y = nullptr) {
    const int R = a.R;
    if (kChain && d >= a.dim && q == 0) s_y[threadIdx.x / kSplit] = 0.0f;
    if (d >= a.dim) return;

    float dl = 0.0f;
    if constexpr (kVecR) {
#pragma unroll
      for (int j = 0; j < kRC; ++j) {
        const int c = q + kSplit * j;
        if (c * E < R) {
          float w[E];
          Chunk<T>::cvt(wv[j], w);
#pragma unroll
          for (int i = 0; i < E; ++i) dl = fmaf(w[i], s_p[c * E + i], dl);
        }
      }
    } else {
      const T* __restrict__ wrow = static_cast<const T*>(a.Wdt) + (size_t)dc * R;
      for (int r = q; r < R; r += kSplit) dl = fmaf(Elem<T>::load1(wrow + r), s_p[r], dl);
    }
    dl = round_to<T>(split_sum(dl));
    const float dt = softplus_t20(dl + (a.dt_bias ? bias_v : 0.0f));
    const float du = dt * u;
    float out = 0.0f;
    float* __restrict__ h = a.state + ((size_t)b * a.dim + dc) * kN + q * kNS;
#pragma unroll
    for (int g = 0; g < kNS / kSV; ++g) {
#pragma unroll
      for (int i = 0; i < kSV; ++i) {
        const int nl = kSV * g + i, n = q * kNS + nl;
        const float av = fast_exp2(-dt * fast_exp2(la[nl] * kLog2e) * kLog2e);  // exp(dt * A), A = -exp(log_A)
        hs[nl] = fmaf(av, hs[nl], du * s_p[R + n]);
        out = fmaf(s_p[R + kN + n], hs[nl], out);
      }
      if constexpr (!kChain) {  // kChain: see store_state
        SV v;
        __builtin_memcpy(&v, &hs[kSV * g], sizeof(v));
        *reinterpret_cast<SV*>(h + kSV * g) = v;
      }
    }
    out = split_sum(out);
    if (q != 0) return;
    out = fmaf(a.Dv ? dv_v : 0.0f, u, out);
    if constexpr (kChain) s_y[threadIdx.x / kSplit] = out * silu_f(z);
    else Elem<T>::store1(static_cast<T*>(a.y) + (size_t)b * a.dim + d, out * silu_f(z));
  }

  // After compute<true>: write the updated state back.  The layer chain calls
  // it after the y hand-off stores, which the other workgroups wait for; the
  // state is read again only at the next token step.
  __device__ __forceinline__ void store_state(const SsmArgs& a) {
    if (d >= a.dim) return;
    float* __restrict__ h = a.state + ((size_t)b * a.dim + dc) * kN + q * kNS;
#pragma unroll
    for (int g = 0; g < kNS / kSV; ++g) {
      SV v;
      __builtin_memcpy(&v, &hs[kSV * g], sizeof(v));
      *reinterpret_cast<SV*>(h + kSV * g) = v;
    }
  }
};

template <typename T, int kN, bool kVecR, bool kParts>
__global__ __launch_bounds__(kDecThreads) void ssm_step_kernel(const SsmArgs a) {
  extern __shared__ __align__(16) float s_p[];  // [nout4] (+ [S][nout4 / 4] float4 with kParts)
  SsmStep<T, kN, kVecR, kParts> st;
  st.begin(a, blockIdx.x, blockIdx.y);
  st.load_parts(a);
  st.load_operands(a);
  st.load_act(a);
  st.finish(a, s_p, reinterpret_cast<float4*>(s_p + a.nout4));
}

// ---------------------------------------------------------------------------
// Layer chain: the token step of every layer of a Mamba stack in one launch.
//
// Per layer the step has three grid-wide dependencies (the in-projection needs
// all of x, the state update the x-projection over all channels, the
// out-projection all of y), so as separate kernels it is three launches per
// layer, each paying launch, ramp and drain (about 4.6 us apiece in a graph,
// for an empty kernel of 256 workgroups) for about a microsecond of memory
// traffic.  Here one persistent grid runs the three phases of every layer in
// turn, with the same GemvWork / SsmStep code as the stand-alone kernels, and
// the workgroups hand activations to each other as LL units:
//
// phase 1 (workgroup i < n1): in-projection rows [16 i, 16 i + 16), norm,
//          conv step and the x-projection partial of the x half: xc (x half)
//          or z (z half) and the partials out as LL units;
// phase 2 (n2 workgroups from the z half on): the state update of 128
//          channels of one batch row from the partials, xc and z: y out as LL
//          units;
// phase 3 (i < n3):        out-projection rows + residual from y: the next
//          layer's input out as LL units (the last layer's to x_out).
//
// Each layer has its own LL buffers, written once per launch, and every unit
// carries the launch's flag (a generation counter the last workgroup out
// advances), so a consumer waits for exactly the units it reads, in one memory
// round trip, with no barrier: a phase starts as soon as its own inputs are
// there.  Each phase's weights and operands are loaded before that wait.
// Every wait is bounded: a workgroup that polls more than maxspin times sets
// the error word and returns; the others see the error word in their polls
// and return too, so the grid always drains, and later launches that find the
// error word set do nothing until the host clears the workspace.
//
// Measured on MI355X before the LL hand-off, with software grid barriers
// between the phases (a group counter per XCD and a root counter, 2.1 us per
// barrier), the chain took 0.99 ms per token at config 4 against 0.92 ms for
// the per-layer kernels: the barriers were half of each layer's 20.6 us.  With
// the LL hand-off, the phase placement and store order described at the
// phases below, LDS operands read before the arithmetic and the state
// update's activations read ahead of its wait, it takes 0.68 ms (14.2 us per
// layer, about 8.5 us of it hand-offs).
struct LayerPtrs {
  const void* w_in;     // (2 dim, K)
  const void* b_in;     // (2 dim) nullable
  const void* norm_w;   // (K)
  const void* conv_w;   // (dim, width)
  const void* conv_b;   // (dim) nullable
  const void* w_x;      // (nout, dim)
  const void* w_dt;     // (dim, R)
  const void* dt_bias;  // (dim) nullable
  const void* log_A;    // (dim, N)
  const void* D;        // (dim) nullable
  const void* w_out;    // (K, dim)
  const void* b_out;    // (K) nullable
  void* window;         // (B, dim, width - 1)
  float* state;         // (B, dim, N) fp32
};

struct LayersArgs {
  const LayerPtrs* layers;  // [nlayers], device memory
  int nlayers, B, K, dim, width, R, nout, nout4, nparts;
  float eps;
  const void* x_in;         // (B, K) input of layer 0
  void* x_out;              // (B, K) output of the last layer
  char* ll;                 // LL buffers: layer l's at ll + l * ll_stride
  size_t ll_stride;
  // byte offsets in a layer's block: its input x (B, K / V units; written by
  // the layer before), the partials (nparts, B, nout4), their slice sums
  // (B, nd, nout4), xc, z and y (B, dim / V)
  uint32_t ll_x, ll_p, ll_q, ll_xc, ll_z, ll_y;
  unsigned* sync;           // generation, done counter and error word
  unsigned maxspin;
};

// sync area: the generation, the done counter and the error word, each in its
// own 256-byte line
constexpr int kSyncLine = 64;
constexpr int kSyncGen = 0, kSyncDone = kSyncLine, kSyncErr = 2 * kSyncLine;
constexpr int kLayersSyncWords = 3 * kSyncLine;

// A pointer read from the layer table is generic to the compiler, which then
// accesses it with flat instructions; flat loads count against the LDS
// counter as well, so every LDS wait would also wait for the prefetched
// weights.  Rebuilding the pointer in the global address space (from its
// integer value, which the compiler cannot fold back to the generic pointer)
// lets it use global instructions; the table holds device memory only.
template <typename P>
__device__ __forceinline__ P* glob(P* p) {
  using G = __attribute__((address_space(1))) P;
  return (P*)((G*)reinterpret_cast<uintptr_t>(p));
}

__device__ __forceinline__ GemvArgs in_proj_args(const LayersArgs& a, const LayerPtrs& L,
                                                 char* lb, unsigned flag) {
  GemvArgs g{};
  g.W = glob(L.w_in); g.x = a.x_in; g.nw = glob(L.norm_w); g.eps = a.eps; g.bias = glob(L.b_in);
  g.res = nullptr; g.y = nullptr; g.B = a.B; g.O = 2 * a.dim; g.K = a.K;
  g.dim = a.dim; g.width = a.width; g.ctx = glob(L.window); g.cw = glob(L.conv_w);
  g.cb = glob(L.conv_b); g.xc = nullptr; g.Wx = glob(L.w_x); g.nout = a.nout; g.nout4 = a.nout4;
  g.part = reinterpret_cast<float*>(lb + a.ll_p); g.flag = flag;
  return g;
}

__device__ __forceinline__ SsmArgs ssm_args(const LayersArgs& a, const LayerPtrs& L, char* lb) {
  SsmArgs s{};
  s.pp = lb + a.ll_p; s.nout = a.nout; s.nout4 = a.nout4; s.nparts = a.nparts; s.R = a.R;
  s.Wdt = glob(L.w_dt); s.dt_bias = glob(L.dt_bias); s.logA = glob(L.log_A); s.Dv = glob(L.D);
  s.xc = lb + a.ll_xc; s.xz = lb + a.ll_z; s.ld_xz = a.dim; s.state = glob(L.state);
  s.y = nullptr; s.dim = a.dim; s.B = a.B;
  return s;
}

__device__ __forceinline__ GemvArgs out_proj_args(const LayersArgs& a, const LayerPtrs& L) {
  GemvArgs g{};
  g.W = glob(L.w_out); g.x = nullptr; g.nw = nullptr; g.eps = a.eps; g.bias = glob(L.b_out);
  g.res = a.x_in; g.y = nullptr; g.B = a.B; g.O = a.K; g.K = a.dim;
  return g;
}

// Phase shapes of the layer chain: 8 waves per workgroup (two per SIMD, so
// each phase's instruction latency is shared out), two rows per wave for the
// in-projection, two K-slices of two rows per wave for the out-projection,
// four threads per channel (4 of the 16 states each) for the state update, so
// that 128 channels per workgroup spread it over twice as many workgroups as
// 256 would (at config 4, 64 instead of 32).
constexpr int kChainWaves = 8;
constexpr int kChainThreads = 64 * kChainWaves;
constexpr int kChainChan = 128;                           // channels per phase-2 workgroup
constexpr int kChainSplit = kChainThreads / kChainChan;   // threads per channel in phase 2
constexpr int kChainKSplit = 2;                            // K-slices of the out-projection
constexpr int kChainRows1 = kXBlock / kChainWaves;         // in-projection rows per wave
constexpr int kChainTaps = 4;                              // conv width limit
constexpr int kChainRC = 8;                                // dt rank up to 8 16-byte chunks

template <typename T, int kMB, int kN, int kRows3>
struct Chain {
  using P1 = GemvWork<T, kMB, kChainRows1, true, kEpiConvX, kChainWaves, 1, 2, kChainTaps>;
  using P2 = SsmStep<T, kN, true, true, kChainSplit, 1, kChainRC, kChainChan>;
  using P3 = GemvWork<T, kMB, kRows3, false, kEpiPlain, kChainWaves, kChainKSplit, 2>;
};

template <typename T, int kMB, int kN, int kRows3>
__global__ __launch_bounds__(kChainThreads) void decode_layers_kernel(const LayersArgs a) {
  using P1 = typename Chain<T, kMB, kN, kRows3>::P1;
  using P2 = typename Chain<T, kMB, kN, kRows3>::P2;
  using P3 = typename Chain<T, kMB, kN, kRows3>::P3;
  constexpr int V = LLVal<T>::V;
  __shared__ struct {
    typename P1::Smem p1;
    typename P3::Smem p3;
  } gsm;
  __shared__ __align__(16) float s_p[kMaxXOut];
  __shared__ float4 s_red[kChainThreads];
  __shared__ float s_y[kChainChan];
  __shared__ unsigned s_flag;
  const int blk = blockIdx.x;
  const int n1 = (2 * a.dim + kXBlock - 1) / kXBlock;
  const int nd = (a.dim + kChainChan - 1) / kChainChan;
  const int n2 = nd * a.B;
  const int n3 = (a.K + P3::kXB - 1) / P3::kXB;
  // workgroups past a GEMV phase's blocks load the last block's operands (read
  // only, never used), so each phase's loads are unconditional
  const int b1 = min(blk, n1 - 1), b3 = min(blk, n3 - 1);
  unsigned* const err = a.sync + kSyncErr;
  // the launch's flag; none (no work) once an earlier launch gave up
  if (threadIdx.x == 0) s_flag = dev_load_u32(err) ? 0u : dev_load_u32(a.sync + kSyncGen) + 1u;
  __syncthreads();
  const unsigned flag = s_flag;
  if (flag == 0) return;
  const LLWait w{flag, a.maxspin, err};
  const size_t xbytes = (size_t)a.B * a.K / V * 8, cbytes = (size_t)a.B * a.dim / V * 8;
  const size_t pbytes = (size_t)a.nparts * a.B * a.nout4 * 8;
  const size_t qbytes = (size_t)a.B * nd * a.nout4 * 8;

  // Each phase's weights and operands go out just before the wait for its
  // input.  (Issuing them a phase earlier, to land during the previous phase's
  // arithmetic, keeps them live there: past 256 VGPRs that spilled and cost
  // 40% at config 4.)
  for (int l = 0; l < a.nlayers; ++l) {
    const LayerPtrs& L = a.layers[l];
    char* lb = a.ll + (size_t)l * a.ll_stride;
    // this layer's input as LL units (layer 0 reads x_in)
    const void* x_ll = l ? lb + a.ll_x : nullptr;
    const GemvArgs g1 = in_proj_args(a, L, lb, flag);
    const SsmArgs s2 = ssm_args(a, L, lb);
    const GemvArgs g3 = out_proj_args(a, L);

    // phase 1: in-projection, conv step, x-projection partials
    P1 p1;
    p1.begin(b1);
    p1.template load_epilogue<true>(g1, gsm.p1);
    p1.load_pass(g1, 0);
    {
      bool ok = true;
      if (l == 0) p1.stage(g1, 0, gsm.p1);
      else ok = p1.stage_ll(g1, x_ll, w, gsm.p1);
      if (__syncthreads_or(!ok)) {
        if (threadIdx.x == 0) dev_store_u32(err, 1u);
        return;
      }
    }
    if (blk < n1) {
      p1.accumulate(g1, 0, gsm.p1);
      p1.template finish<true>(g1, gsm.p1);
      __syncthreads();
      // xc (x half) or z (z half) of the workgroup's 16 channels as LL units
      const int r0 = blk * kXBlock;
      const bool xh = r0 < a.dim;
      const int c0 = xh ? r0 : r0 - a.dim;
      constexpr int kU = kXBlock / V;
      if ((int)threadIdx.x < a.B * kU) {
        const int bb = threadIdx.x / kU, uu = threadIdx.x % kU;
        const float* src = xh ? gsm.p1.xc[bb] : gsm.p1.yt[bb];
        ll_put(dev_rsrc(lb + (xh ? a.ll_xc : a.ll_z), cbytes),
               (uint32_t)((bb * a.dim + c0) / V + uu),
               LLVal<T>::pack(src[uu * V], src[(uu * V + 1) % kXBlock]), flag);
      }
      // the conv cache after the hand-off stores (stores issue in order, so
      // cache writes issued first would hold up the units others wait for)
      p1.store_window(g1);
    }

    // phase 2: partial sums, dt projection, state update, gate.  The first
    // ns of the nd workgroups of a batch row each sum one ns-th of its partial
    // blocks (in block order) and publish those slice sums; each of the nd then
    // adds the ns slice sums (in slice order): two small hand-offs instead of
    // every workgroup reading all of its row's partial blocks.  Phase 2 runs on the
    // workgroups of phase 1's z half (from z2 on) where there are enough of
    // them: they finish phase 1 earlier (no conv step or x-projection
    // partials), so their phase-2 operand loads are in before the partials
    // arrive and the wait for the partials is not held up behind them.
    const int z2 = max(0, min(a.dim / kXBlock, (int)gridDim.x - n2));
    if (blk - z2 >= 0 && blk - z2 < n2) {
      const int blk2 = blk - z2;
      const int bb = blk2 / nd, dblk = blk2 % nd, d0 = dblk * kChainChan;
      const int ng = a.nout4 / 4;
      P2 p2;
      p2.begin(s2, dblk, bb);
      p2.load_operands(s2);
      // ns slices of the partial blocks, one per workgroup dblk < ns (every
      // workgroup then reads all ns slice sums in one round: ns ng <= threads)
      const int ns = min(nd, kChainThreads / ng);
      if (dblk < ns) {
        const int w_lo = dblk * a.nparts / ns, nw = (dblk + 1) * a.nparts / ns - w_lo;
        {
          const int t = threadIdx.x, wl = t / ng, gi = t - wl * ng;
          const uint32_t u0 = (uint32_t)(((w_lo + min(wl, nw - 1)) * a.B + bb) * a.nout4 + 4 * gi);
          const uint32_t pairs[2] = {u0, u0 + 2};
          u32x4_v v[2];
          const bool ok = ll_wait2<2>(dev_rsrc(lb + a.ll_p, pbytes), pairs, wl < nw, w, v);
          if (wl < nw)
            s_red[t] = make_float4(__uint_as_float(v[0][0]), __uint_as_float(v[0][2]),
                                   __uint_as_float(v[1][0]), __uint_as_float(v[1][2]));
          if (__syncthreads_or(!ok)) {
            if (threadIdx.x == 0) dev_store_u32(err, 1u);
            return;
          }
        }
        if ((int)threadIdx.x < a.nout4) {
          const int jc = threadIdx.x;
          const float* r = reinterpret_cast<const float*>(s_red) + jc;
          float t = 0.0f;
          for (int w0 = 0; w0 < nw; w0 += 4) {  // 4 reads in flight, then the adds in order
            float rv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) rv[i] = r[min(w0 + i, nw - 1) * a.nout4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (w0 + i < nw) t += rv[i];
          }
          ll_put(dev_rsrc(lb + a.ll_q, qbytes), (uint32_t)((bb * nd + dblk) * a.nout4 + jc),
                 __float_as_uint(t), flag);
        }
      }
      {
        const int t = threadIdx.x, sl = t / ng, gi = t - sl * ng;
        const uint32_t u0 = (uint32_t)((bb * nd + min(sl, ns - 1)) * a.nout4 + 4 * gi);
        const uint32_t pairs[2] = {u0, u0 + 2};
        u32x4_v v[2];
        p2.issue_act_ll(s2);
        const bool ok_q = ll_wait2<2>(dev_rsrc(lb + a.ll_q, qbytes), pairs, sl < ns, w, v);
        const bool ok_a = p2.load_act_ll(s2, w);
        __syncthreads();  // every thread is done with the slice sums in s_red
        if (sl < ns)
          s_red[t] = make_float4(__uint_as_float(v[0][0]), __uint_as_float(v[0][2]),
                                 __uint_as_float(v[1][0]), __uint_as_float(v[1][2]));
        if (__syncthreads_or(!(ok_q && ok_a))) {
          if (threadIdx.x == 0) dev_store_u32(err, 1u);
          return;
        }
      }
      if ((int)threadIdx.x < a.nout) {
        const float* r = reinterpret_cast<const float*>(s_red) + threadIdx.x;
        float t = 0.0f;
        for (int s0 = 0; s0 < ns; s0 += 4) {  // 4 reads in flight, then the adds in order
          float rv[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) rv[i] = r[min(s0 + i, ns - 1) * a.nout4];
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (s0 + i < ns) t += rv[i];
        }
        s_p[threadIdx.x] = round_to<T>(t);
      }
      __syncthreads();
      p2.template compute<true>(s2, s_p, s_y);
      __syncthreads();
      constexpr int kU = kChainChan / V;
      if ((int)threadIdx.x < kU && d0 + (int)threadIdx.x * V < a.dim) {
        const int i = threadIdx.x * V;
        ll_put(dev_rsrc(lb + a.ll_y, cbytes), (uint32_t)((bb * a.dim + d0) / V + threadIdx.x),
               LLVal<T>::pack(s_y[i], s_y[(i + 1) % kChainChan]), flag);
      }
      p2.store_state(s2);  // the SSM state after the y hand-off stores
    }

    // phase 3: out-projection + residual -> the next layer's input
    P3 p3;
    p3.begin(b3);
    p3.template load_epilogue<true>(g3, gsm.p3, x_ll);
    p3.load_pass(g3, 0);
    {
      const bool ok = blk < n3 ? p3.stage_ll(g3, lb + a.ll_y, w, gsm.p3) : true;
      if (__syncthreads_or(!ok)) {
        if (threadIdx.x == 0) dev_store_u32(err, 1u);
        return;
      }
    }
    if (blk < n3) {
      p3.accumulate(g3, 0, gsm.p3);
      p3.template finish<true>(g3, gsm.p3);
      __syncthreads();
      const int r0 = blk * P3::kXB;
      if (l + 1 == a.nlayers) {
        if ((int)threadIdx.x < a.B * P3::kXB) {
          const int bb = threadIdx.x / P3::kXB, rr = threadIdx.x % P3::kXB;
          if (r0 + rr < a.K)
            Elem<T>::store1(static_cast<T*>(a.x_out) + (size_t)bb * a.K + r0 + rr, gsm.p3.yt[bb][rr]);
        }
      } else {
        constexpr int kU = P3::kXB / V;
        if ((int)threadIdx.x < a.B * kU) {
          const int bb = threadIdx.x / kU, uu = threadIdx.x % kU;
          const float* src = gsm.p3.yt[bb];
          ll_put(dev_rsrc(a.ll + (size_t)(l + 1) * a.ll_stride + a.ll_x, xbytes),
                 (uint32_t)((bb * a.K + r0) / V + uu),
                 LLVal<T>::pack(src[uu * V], src[(uu * V + 1) % P3::kXB]), flag);
        }
      }
    }
  }
  // the last workgroup out advances the generation (every other one has
  // passed all of its waits by then); flags run over [1, 2^32 - 2]
  if (threadIdx.x == 0 && dev_add_u32(a.sync + kSyncDone, 1u) == gridDim.x - 1) {
    dev_store_u32(a.sync + kSyncDone, 0u);
    dev_store_u32(a.sync + kSyncGen, flag == 0xFFFFFFFEu ? 0u : flag);
  }
}

// ---------------------------------------------------------------------------
// Greedy pick of the decode loop: token[b] = argmax_v p[b, v], the first
// maximum (NaN ranks above every number, as in torch.argmax) -- the argmax of
// models/causal_lm.py:117-120 applied to the softmax output -- and the loop's
// bookkeeping: tokens[b, min(pos, cols - 1)] = token[b], then pos += 1.
//
// kPickParts workgroups per row each find the best (value, index) of a slice
// and store it at device scope; the last workgroup to finish (a device-scope
// counter, which it clears again) combines the slices and does the
// bookkeeping.  (value, index) pairs are totally ordered (indexes differ), so
// the result does not depend on the order of the combination.
constexpr int kPickThreads = 256;
constexpr int kPickParts = 32;

// (v, i) ranks before (w, j)
__device__ __forceinline__ bool pick_beats(float v, int i, float w, int j) {
  const bool vn = v != v, wn = w != w;
  if (vn != wn) return vn;
  if (!vn && v != w) return v > w;
  return i < j;
}

__device__ __forceinline__ void pick_reduce_wave(float& v, int& i) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ov = __shfl_xor(v, m, 64);
    const int oi = __shfl_xor(i, m, 64);
    if (pick_beats(ov, oi, v, i)) { v = ov; i = oi; }
  }
}

// ws: [0] the counter, then from word 64 the slices' (value bits, index)
template <typename T>
__global__ __launch_bounds__(kPickThreads) void pick_kernel(const T* __restrict__ p, int B, int V,
                                                            int64_t* __restrict__ token,
                                                            int64_t* __restrict__ tokens,
                                                            int64_t ld, int64_t cols,
                                                            int64_t* __restrict__ pos,
                                                            unsigned* __restrict__ ws) {
  constexpr int E = Chunk<T>::E;
  constexpr int kIn = 4;  // chunks per thread in flight
  using Raw = typename Chunk<T>::Raw;
  __shared__ float s_v[kPickThreads / 64];
  __shared__ int s_i[kPickThreads / 64];
  __shared__ int s_last;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = blockIdx.x / kPickParts, part = blockIdx.x % kPickParts;
  const int nc = V / E;  // rows are whole chunks
  const int c_lo = part * nc / kPickParts, c_hi = (part + 1) * nc / kPickParts;
  const T* __restrict__ row = p + (size_t)b * V;
  float bv = -INFINITY;
  int bi = V;  // ranks after every real index
  for (int c0 = c_lo; c0 < c_hi; c0 += kPickThreads * kIn) {
    Raw r[kIn];  // all of the round's loads first (clamped addresses, used when in range)
#pragma unroll
    for (int j = 0; j < kIn; ++j)
      r[j] = ldchunk(row + (size_t)min(c0 + j * kPickThreads + (int)threadIdx.x, nc - 1) * E);
#pragma unroll
    for (int j = 0; j < kIn; ++j) {
      const int c = c0 + j * kPickThreads + threadIdx.x;
      if (c < c_hi) {
        float f[E];
        Chunk<T>::cvt(r[j], f);
#pragma unroll
        for (int k = 0; k < E; ++k)
          if (pick_beats(f[k], c * E + k, bv, bi)) { bv = f[k]; bi = c * E + k; }
      }
    }
  }
  pick_reduce_wave(bv, bi);
  if (lane == 0) { s_v[wave] = bv; s_i[wave] = bi; }
  __syncthreads();
  const auto r = dev_rsrc(ws, (size_t)(64 + 2 * B * kPickParts) * 4);
  if (threadIdx.x == 0) {
    float v = s_v[0];
    int i = s_i[0];
    for (int w = 1; w < kPickThreads / 64; ++w)
      if (pick_beats(s_v[w], s_i[w], v, i)) { v = s_v[w]; i = s_i[w]; }
    const u32x2_v pr = {__float_as_uint(v), (uint32_t)i};
    __builtin_amdgcn_raw_buffer_store_b64(pr, r, (int)((64 + 2 * blockIdx.x) * 4), 0, kSC1);
    // release: the slice is visible at device scope before it is counted;
    // acquire: the last workgroup sees every other workgroup's slice
    s_last = __hip_atomic_fetch_add(ws, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) ==
             gridDim.x - 1;
  }
  __syncthreads();
  if (!s_last) return;
  // every thread of the last workgroup reads slices: order its loads after
  // the counter as well (the barrier orders them only within the workgroup)
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  // the last workgroup: wave w combines rows w, w + 4, ... (no barrier inside)
  const int64_t ps = pos ? *pos : 0;
  const int64_t col = ps < cols - 1 ? ps : cols - 1;
  for (int rb = wave; rb < B; rb += kPickThreads / 64) {
    float v = -INFINITY;
    int i = V;
    if (lane < kPickParts) {
      const u32x2_v pr =
          __builtin_amdgcn_raw_buffer_load_b64(r, (int)((64 + 2 * (rb * kPickParts + lane)) * 4), 0, kSC1);
      v = __uint_as_float(pr[0]);
      i = (int)pr[1];
    }
    pick_reduce_wave(v, i);
    if (lane == 0) {
      token[rb] = i;
      if (tokens) tokens[(size_t)rb * ld + col] = i;
    }
  }
  __syncthreads();  // every lane has read pos
  if (threadIdx.x == 0) {
    if (pos) *pos = ps + 1;
    dev_store_u32(ws, 0u);  // the counter, for the next launch
  }
}

template <typename T, int kMB, int kRows>
hipError_t launch_gemv_r(const GemvArgs& a, bool norm, bool conv, hipStream_t st) {
  const int rows_per_block = (kDecThreads / 64) * kRows;
  const dim3 grid((a.O + rows_per_block - 1) / rows_per_block);
  if (conv && a.Wx) {
    if constexpr (kRows == kXRows) {
      if (norm)
        hipLaunchKernelGGL((gemv_kernel<T, kMB, kRows, true, kEpiConvX>), grid, dim3(kDecThreads), 0, st, a);
      else
        hipLaunchKernelGGL((gemv_kernel<T, kMB, kRows, false, kEpiConvX>), grid, dim3(kDecThreads), 0, st, a);
    } else {
      return hipErrorInvalidValue;
    }
  } else if (conv) {
    if (norm)
      hipLaunchKernelGGL((gemv_kernel<T, kMB, kRows, true, kEpiConv>), grid, dim3(kDecThreads), 0, st, a);
    else
      hipLaunchKernelGGL((gemv_kernel<T, kMB, kRows, false, kEpiConv>), grid, dim3(kDecThreads), 0, st, a);
  } else {
    if (norm)
      hipLaunchKernelGGL((gemv_kernel<T, kMB, kRows, true, kEpiPlain>), grid, dim3(kDecThreads), 0, st, a);
    else
      hipLaunchKernelGGL((gemv_kernel<T, kMB, kRows, false, kEpiPlain>), grid, dim3(kDecThreads), 0, st, a);
  }
  return hipGetLastError();
}

// rows per wave of a GEMV: four for tall matrices (the LM head) and with the
// x-projection partials, one for short ones (more workgroups in flight), two
// otherwise
inline int gemv_rows(int O, bool conv, bool xproj) {
  if (O >= 16384 || (conv && xproj)) return 4;
  if (O <= 2048 && !conv) return 1;
  return 2;
}

template <typename T, int kMB>
hipError_t launch_gemv_b(const GemvArgs& a, bool norm, bool conv, hipStream_t st) {
  switch (gemv_rows(a.O, conv, a.Wx != nullptr)) {
    case 4: return launch_gemv_r<T, kMB, 4>(a, norm, conv, st);
    case 1: return launch_gemv_r<T, kMB, 1>(a, norm, conv, st);
    default: return launch_gemv_r<T, kMB, 2>(a, norm, conv, st);
  }
}

template <typename T>
hipError_t launch_gemv_t(const GemvArgs& a, bool norm, bool conv, hipStream_t st) {
  if (a.B <= 1) return launch_gemv_b<T, 1>(a, norm, conv, st);
  if (a.B <= 2) return launch_gemv_b<T, 2>(a, norm, conv, st);
  if (a.B <= 4) return launch_gemv_b<T, 4>(a, norm, conv, st);
  return launch_gemv_b<T, 8>(a, norm, conv, st);
}

template <typename T, int kN>
hipError_t launch_ssm_step_n(const SsmArgs& a, bool vecR, hipStream_t st) {
  const dim3 grid((a.dim + kDecThreads - 1) / kDecThreads, a.B);
  // s_p, plus the partial sums' [S][nout4 / 4] float4 with partials (S * nout4 <= 4 * 256)
  const size_t lds = (size_t)a.nout4 * sizeof(float) +
                     (a.nparts ? (size_t)(kDecThreads / (a.nout4 / 4)) * a.nout4 * sizeof(float) : 0);
#define SSM_STEP_LAUNCH(vr, pt) \
  hipLaunchKernelGGL((ssm_step_kernel<T, kN, vr, pt>), grid, dim3(kDecThreads), lds, st, a)
  if (a.nparts) {
    if (vecR) SSM_STEP_LAUNCH(true, true);
    else SSM_STEP_LAUNCH(false, true);
  } else {
    if (vecR) SSM_STEP_LAUNCH(true, false);
    else SSM_STEP_LAUNCH(false, false);
  }
#undef SSM_STEP_LAUNCH
  return hipGetLastError();
}

template <typename T>
hipError_t launch_ssm_step_t(const SsmArgs& a, int nstate, bool vecR, hipStream_t st) {
  switch (nstate) {
    case 4: return launch_ssm_step_n<T, 4>(a, vecR, st);
    case 8: return launch_ssm_step_n<T, 8>(a, vecR, st);
    case 16: return launch_ssm_step_n<T, 16>(a, vecR, st);
    case 32: return launch_ssm_step_n<T, 32>(a, vecR, st);
    case 64: return launch_ssm_step_n<T, 64>(a, vecR, st);
    default: return hipErrorInvalidValue;
  }
}

// out-projection rows per wave of the layer chain.  Two rows (8 per
// workgroup) rather than one: every out-projection workgroup reads all of y,
// so half as many of them halve that hand-off's reads (at config 4, 4 MB
// instead of 8 MB per layer), and the workgroups past them skip the phase.
constexpr int kChainRows3 = 2;

// workgroups the layer chain runs with: the largest of its three phases
int layers_grid(int B, int K, int dim) {
  const int n1 = (2 * dim + kXBlock - 1) / kXBlock;
  const int n2 = ((dim + kChainChan - 1) / kChainChan) * B;
  const int rows = (kChainWaves / kChainKSplit) * kChainRows3;
  const int n3 = (K + rows - 1) / rows;
  return std::max(n1, std::max(n2, n3));
}

// Largest grid of `kernel` whose workgroups are all resident at once on the
// current device (the layer chain's waits need every workgroup running).
hipError_t resident_limit(const void* kernel, int* limit) {
  int dev = 0, cus = 0, per_cu = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kChainThreads, 0);
  *limit = cus * per_cu;
  return e;
}

template <typename T, int kMB, int kN, int kRows3>
hipError_t launch_layers_k(const LayersArgs& a, hipStream_t st) {
  const void* fn = reinterpret_cast<const void*>(&decode_layers_kernel<T, kMB, kN, kRows3>);
  // resident-grid limit per device, queried once (the occupancy query is a host call)
  static int limit[64] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  if (limit[dev] == 0) {
    int lim = 0;
    if ((e = resident_limit(fn, &lim)) != hipSuccess) return e;
    limit[dev] = lim;
  }
  const int G = layers_grid(a.B, a.K, a.dim);
  if (G > limit[dev]) return hipErrorCooperativeLaunchTooLarge;
  hipLaunchKernelGGL((decode_layers_kernel<T, kMB, kN, kRows3>), dim3(G), dim3(kChainThreads), 0, st, a);
  return hipGetLastError();
}

template <typename T, int kMB>
hipError_t launch_layers_b(const LayersArgs& a, hipStream_t st) {
  return launch_layers_k<T, kMB, 16, kChainRows3>(a, st);
}

template <typename T>
hipError_t launch_layers_t(const LayersArgs& a, hipStream_t st) {
  if (a.B <= 1) return launch_layers_b<T, 1>(a, st);
  if (a.B <= 2) return launch_layers_b<T, 2>(a, st);
  if (a.B <= 4) return launch_layers_b<T, 4>(a, st);
  return launch_layers_b<T, 8>(a, st);
}

// Why the layer chain cannot run a shape (nullptr: it can).  Each GEMV phase
// runs in one pass (its prefetched weights are the whole row slice), and each
// state-update thread waits for all of its partial blocks in one round.
template <typename T>
const char* layers_unsupported_t(int K, int dim, int nout) {
  using C = Chain<T, 1, 16, 1>;
  if (K > C::P1::PK) return "model_dim exceeds the in-projection's single pass";
  if (dim > C::P3::PK) return "dim exceeds the out-projection's single pass";
  const int ng = ((nout + 3) & ~3) / 4;
  const int nd = (dim + kChainChan - 1) / kChainChan;
  const int ns = std::min(nd, kChainThreads / ng);
  const int nparts = dim / kXBlock;
  if (ns < 1 || ((nparts + ns - 1) / ns) * ng > kChainThreads)
    return "too many x-projection partial blocks per state-update workgroup";
  return nullptr;
}

}  // namespace

int decode_max_batch() { return kMaxDecBatch; }

int decode_xproj_blocks(int64_t dim, int64_t nout) {
  if (dim < kXBlock || dim % kXBlock || nout < 1 || nout > kMaxXOut) return 0;
  return (int)(dim / kXBlock);
}

hipError_t launch_decode_gemv(int bf16, const void* W, const void* x, const void* nw, float eps,
                              const void* bias, const void* res, void* y, int B, int O, int K,
                              hipStream_t st) {
  ProfScope prof("decode_gemv", st);
  GemvArgs a{};
  a.W = W; a.x = x; a.nw = nw; a.eps = eps; a.bias = bias; a.res = res; a.y = y;
  a.B = B; a.O = O; a.K = K;
  return bf16 ? launch_gemv_t<__hip_bfloat16>(a, nw != nullptr, false, st)
              : launch_gemv_t<float>(a, nw != nullptr, false, st);
}

hipError_t launch_decode_in_proj_conv(int bf16, const void* W, const void* x, const void* nw,
                                      float eps, const void* bias, void* xz, int B, int dim, int K,
                                      int width, void* ctx, const void* cw, const void* cb,
                                      void* xc, const void* Wx, int nout, float* part,
                                      hipStream_t st) {
  ProfScope prof("decode_in_proj_conv", st);
  GemvArgs a{};
  a.W = W; a.x = x; a.nw = nw; a.eps = eps; a.bias = bias; a.res = nullptr; a.y = xz;
  a.B = B; a.O = 2 * dim; a.K = K;
  a.dim = dim; a.width = width; a.ctx = ctx; a.cw = cw; a.cb = cb; a.xc = xc;
  a.Wx = Wx; a.nout = nout; a.nout4 = (nout + 3) & ~3; a.part = part;
  return bf16 ? launch_gemv_t<__hip_bfloat16>(a, nw != nullptr, true, st)
              : launch_gemv_t<float>(a, nw != nullptr, true, st);
}

hipError_t launch_decode_ssm_step(int bf16, const void* p, int nout, int nparts, int R,
                                  const void* Wdt, const void* dtb, const void* logA, const void* D,
                                  const void* xc, const void* xz, int ld, float* state, void* y,
                                  int B, int dim, int nstate, bool vecR, hipStream_t st) {
  ProfScope prof("decode_ssm_step", st);
  SsmArgs a{};
  a.pp = p; a.nout = nout; a.nout4 = (nout + 3) & ~3; a.nparts = nparts; a.R = R;
  a.Wdt = Wdt; a.dt_bias = dtb; a.logA = logA; a.Dv = D; a.xc = xc; a.xz = xz; a.ld_xz = ld;
  a.state = state; a.y = y; a.dim = dim; a.B = B;
  return bf16 ? launch_ssm_step_t<__hip_bfloat16>(a, nstate, vecR, st)
              : launch_ssm_step_t<float>(a, nstate, vecR, st);
}

// workspace of the layer chain: the sync area, then per layer a block of LL
// buffers (8-byte units of 4 data bytes): the layer's input x, the partials,
// their slice sums, xc, z and y, each 256-byte aligned
namespace {
struct LayersWs {
  size_t ll, stride, x, p, q, xc, z, y, total;
};

LayersWs layers_ws(int B, int nlayers, int K, int dim, int nout, int elem) {
  auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
  const size_t V = 4 / elem;
  LayersWs w{};
  w.ll = up(kLayersSyncWords * sizeof(unsigned));
  size_t o = 0;
  w.x = o; o += up((size_t)B * K / V * 8);
  w.p = o; o += up((size_t)(dim / kXBlock) * B * ((nout + 3) & ~3) * 8);
  w.q = o; o += up((size_t)B * ((dim + kChainChan - 1) / kChainChan) * ((nout + 3) & ~3) * 8);
  w.xc = o; o += up((size_t)B * dim / V * 8);
  w.z = o; o += up((size_t)B * dim / V * 8);
  w.y = o; o += up((size_t)B * dim / V * 8);
  w.stride = o;
  w.total = w.ll + (size_t)nlayers * w.stride;
  return w;
}
}  // namespace

int64_t decode_layers_workspace(int B, int nlayers, int K, int dim, int nout, int bf16) {
  return (int64_t)layers_ws(B, nlayers, K, dim, nout, bf16 ? 2 : 4).total;
}

const char* decode_layers_unsupported(int K, int dim, int nout, int bf16) {
  return bf16 ? layers_unsupported_t<__hip_bfloat16>(K, dim, nout)
              : layers_unsupported_t<float>(K, dim, nout);
}

int64_t decode_layers_error_offset() { return (int64_t)kSyncErr * sizeof(unsigned); }
static_assert(kSyncErr * sizeof(unsigned) == 512, "the error word's offset is part of the ABI");

int64_t decode_pick_workspace(int B) { return (int64_t)(64 + 2 * B * kPickParts) * 4; }

hipError_t launch_decode_pick(int bf16, const void* p, int B, int V, int64_t* token,
                              int64_t* tokens, int64_t ld, int64_t cols, int64_t* pos, void* ws,
                              hipStream_t st) {
  ProfScope prof("decode_pick", st);
  const dim3 grid(B * kPickParts);
  unsigned* w = static_cast<unsigned*>(ws);
  if (bf16)
    hipLaunchKernelGGL(pick_kernel<__hip_bfloat16>, grid, dim3(kPickThreads), 0, st,
                       static_cast<const __hip_bfloat16*>(p), B, V, token, tokens, ld, cols, pos, w);
  else
    hipLaunchKernelGGL(pick_kernel<float>, grid, dim3(kPickThreads), 0, st,
                       static_cast<const float*>(p), B, V, token, tokens, ld, cols, pos, w);
  return hipGetLastError();
}

int decode_layers_grid(int B, int K, int dim) { return layers_grid(B, K, dim); }

int decode_layers_max_width() { return kChainTaps; }

hipError_t launch_decode_layers(int bf16, const void* table, int nlayers, int B, int K, int dim,
                                int width, int R, int nout, float eps, const void* x, void* out,
                                void* ws, hipStream_t st) {
  ProfScope prof("decode_layers", st);
  const LayersWs w = layers_ws(B, nlayers, K, dim, nout, bf16 ? 2 : 4);
  char* base = static_cast<char*>(ws);
  LayersArgs a{};
  a.layers = static_cast<const LayerPtrs*>(table);
  a.nlayers = nlayers; a.B = B; a.K = K; a.dim = dim; a.width = width; a.R = R;
  a.nout = nout; a.nout4 = (nout + 3) & ~3; a.nparts = dim / kXBlock; a.eps = eps;
  a.x_in = x; a.x_out = out;
  a.ll = base + w.ll; a.ll_stride = w.stride;
  a.ll_x = (uint32_t)w.x; a.ll_p = (uint32_t)w.p; a.ll_q = (uint32_t)w.q; a.ll_xc = (uint32_t)w.xc;
  a.ll_z = (uint32_t)w.z; a.ll_y = (uint32_t)w.y;
  a.sync = reinterpret_cast<unsigned*>(base);
  // about a second of polling at most (a poll is a device-memory round trip)
  a.maxspin = 1u << 20;
  return bf16 ? launch_layers_t<__hip_bfloat16>(a, st) : launch_layers_t<float>(a, st);
}

}  // namespace ssm
