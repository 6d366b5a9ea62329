// Selective-scan backward for gfx950.
//
// Gradients (reference semantics: csrc/selective_scan/backward_kernel.cu:212-452),
// with G_t the adjoint of h_t and gamma_t = a_{t+1} G_{t+1} its part coming
// from later steps (gamma_{L-1} = dh_last):
//   G_t      = gamma_t + dout_t * C_t
//   du_t     = D * dout_t + delta_t * sum_n G_t B_t
//   ddelta_t = softplus'(x_t) * (u_t * sum_n G_t B_t + sum_n A_n G_t a_t h_{t-1})
//   dA_n    += sum_t delta_t G_t a_t h_{t-1}         (over b and t)
//   dB[b,n,t] = sum_d G_t delta_t u_t,   dC[b,n,t] = sum_d dout_t h_t
//   dD       = sum dout * u,  dbias = sum ddelta,  dh_init = gamma_{-1}
// dout is the upstream gradient masked to zero at padded positions (the loss
// does not see them), times silu(z) when the z gate is fused; then
// dz = dy * out * silu'(z) with out recomputed from the states.
//
// Work decomposition mirrors the forward (workgroup = batch row b x 64
// channels, 4 waves, lane = channel, wave w = state group G = g*4 + w).  Tiles
// of kTileBwd steps are walked from the end; inside a tile, 16-step sub-chunks are
// walked from the end.  For each sub-chunk the wave reloads the state saved by
// the forward at the sub-chunk start, recomputes the 16 states and decay
// factors into registers, then runs the reverse recurrence.  Per-position sums
// over states (sum G B, sum A G a h, sum C h) leave each wave in its own LDS
// slice and are added in a fixed order; the per-position sums over channels
// (dB, dC) are reduced across the
// 64 lanes with a permlane/DPP reduce-scatter and written as one partial per
// (channel block, b, n, t), which a second small kernel adds up.  dA, dD and
// dbias are written as per-batch-row partials reduced by the same kernel, so
// the result is deterministic (no global atomics).
#include "ss_io.cuh"
#include "ss_params.h"
#include "ss_prof.h"

namespace ssm {

template <typename T, int kSG, bool kHasZ, bool kAligned>
__global__ __launch_bounds__(256) void scan_bwd_kernel(
    const ScanDims p, const T* __restrict__ u, const T* __restrict__ dl,
    const float* __restrict__ Ap, const float* __restrict__ bc,
    const float* __restrict__ Dp, const float* __restrict__ biasp,
    const float* __restrict__ h_init, const int64_t* __restrict__ length,
    const T* __restrict__ zp, const float* __restrict__ h_chunks, const T* __restrict__ dyp,
    const float* __restrict__ dh_last, T* __restrict__ dup, T* __restrict__ ddp,
    T* __restrict__ dzp, float* __restrict__ dh_init, float* __restrict__ ws_bc,
    float* __restrict__ ws_A, float* __restrict__ ws_D, float* __restrict__ ws_bias) {
  using E = Elem<T>;
  constexpr int kWaves = 4;
  constexpr int kThreads = 64 * kWaves;
  constexpr int kTile = kTileBwd;
  constexpr int kVec = E::kVec;
  constexpr int kLPR = kTile / kVec;
  constexpr int kRPP = kThreads / kLPR;
  constexpr int kPasses = kBlockCh / kRPP;
  constexpr int kT4 = kTile / 4;
  constexpr int kSub = kChunk;          // 16 steps per sub-chunk
  constexpr int kStride = kTile + 1;    // padded row of the [channel][step] LDS sums
  constexpr int kSlice = kBlockCh * kStride;

  __shared__ float4 sDelta[kT4][kBlockCh];  // delta (0 at padded steps)
  __shared__ float4 sDu[kT4][kBlockCh];     // delta * u
  __shared__ float4 sDout[kT4][kBlockCh];   // masked dout (after the z gate)
  __shared__ float4 sU[kT4][kBlockCh];
  __shared__ float4 sX[kT4][kBlockCh];      // delta_raw + bias
  // one slice per wave of the per-position sums over that wave's states; the
  // slices are added in a fixed order in phase C (deterministic result)
  __shared__ float sGB[kWaves * kSlice];   // sum_n G B
  __shared__ float sDD[kWaves * kSlice];   // sum_n A G a h_{t-1}
  __shared__ float sY[kHasZ ? kWaves * kSlice : 1];  // sum_n C h

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = wave_id_uniform();
  const int b = blockIdx.y;
  const int blk = blockIdx.x;
  const int d0 = blk * kBlockCh;
  const int L = p.seqlen, Dm = p.dim, N = p.nstate;
  const int ngroups = (N + 3) / 4;
  const int Lp = bc_row_len(L);
  const size_t rb = (size_t)b * Dm;
  const size_t nBC = (size_t)p.batch * N * L;

  int vlo, vhi;
  valid_window(length, p.pad_right, b, L, vlo, vhi);

  const int ch = d0 + lane;
  const bool ch_ok = ch < Dm;

  // persistent per-state values: reverse carry gamma and dA accumulator
  float gam[kSG][4], dA[kSG][4];
#pragma unroll
  for (int g = 0; g < kSG; ++g)
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int n = (g * kWaves + w) * 4 + s;
      const bool ok = ch_ok && n < N;
      gam[g][s] = (ok && dh_last) ? dh_last[(rb + ch) * N + n] : 0.0f;
      dA[g][s] = 0.0f;
    }

  const int a_row = tid / kLPR;
  const int a_col = (tid % kLPR) * kVec;
  float Dv[kPasses], Bias[kPasses], accD[kPasses], accB[kPasses];
#pragma unroll
  for (int ps = 0; ps < kPasses; ++ps) {
    const int c = d0 + a_row + ps * kRPP;
    Dv[ps] = (c < Dm && Dp) ? Dp[c] : 0.0f;
    Bias[ps] = (c < Dm && biasp) ? biasp[c] : 0.0f;
    accD[ps] = 0.0f;
    accB[ps] = 0.0f;
  }
  const bool softplus = p.softplus != 0;

  float* const wGB = sGB + w * kSlice;
  float* const wDD = sDD + w * kSlice;
  float* const wY = sY + (kHasZ ? w * kSlice : 0);

  const int ntiles = (L + kTile - 1) / kTile;
  for (int tile = ntiles - 1; tile >= 0; --tile) {
    const int t0 = tile * kTile;
    // ---- phase A: stage per-position quantities
    float dzf[kHasZ ? kPasses : 1][kVec];  // dy_masked * silu'(z), times out later
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) {
      const int row = a_row + ps * kRPP;
      const int c = d0 + row;
      const int t = t0 + a_col;
      const bool ok = c < Dm;
      float uv[kVec], dv[kVec], yv[kVec];
      load_row<T, kAligned>(u + (rb + c) * L, t, L, ok, uv);
      load_row<T, kAligned>(dl + (rb + c) * L, t, L, ok, dv);
      load_row<T, kAligned>(dyp + (rb + c) * L, t, L, ok, yv);
      float zv[kVec];
      if constexpr (kHasZ) load_row<T, kAligned>(zp + (rb + c) * L, t, L, ok, zv);
      float de[kVec], du[kVec], dov[kVec], xv[kVec];
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        const float x = dv[j] + Bias[ps];
        const float dt = softplus ? softplus_t20(x) : x;
        const int tt = t + j;
        const bool valid = tt >= vlo && tt < vhi;
        de[j] = valid ? dt : 0.0f;
        du[j] = de[j] * uv[j];
        const float dym = valid ? yv[j] : 0.0f;
        if constexpr (kHasZ) {
          dov[j] = dym * silu_f(zv[j]);
          dzf[ps][j] = dym * silu_grad_f(zv[j]);
        } else {
          dov[j] = dym;
        }
        xv[j] = x;
      }
#pragma unroll
      for (int q = 0; q < kVec / 4; ++q) {
        const int t4 = a_col / 4 + q;
        sDelta[t4][row] = make_float4(de[4 * q], de[4 * q + 1], de[4 * q + 2], de[4 * q + 3]);
        sDu[t4][row] = make_float4(du[4 * q], du[4 * q + 1], du[4 * q + 2], du[4 * q + 3]);
        sDout[t4][row] = make_float4(dov[4 * q], dov[4 * q + 1], dov[4 * q + 2], dov[4 * q + 3]);
        sU[t4][row] = make_float4(uv[4 * q], uv[4 * q + 1], uv[4 * q + 2], uv[4 * q + 3]);
        sX[t4][row] = make_float4(xv[4 * q], xv[4 * q + 1], xv[4 * q + 2], xv[4 * q + 3]);
      }
    }
    __syncthreads();

    // ---- phase B: sub-chunks from the end of the tile
    const int nsub = min(kTile / kSub, (L - t0 + kSub - 1) / kSub);
    for (int k = nsub - 1; k >= 0; --k) {
      const int ts = t0 + k * kSub;  // first step of the sub-chunk
      const int c = ts / kChunk;     // its chunk index
#pragma unroll
      for (int g = 0; g < kSG; ++g) {
        const int G = g * kWaves + w;
        if (G >= ngroups) {  // wave-uniform; a wave with no states leaves zeros
          if (g == 0) {
#pragma unroll
            for (int i = 0; i < kSub; ++i) {
              const int li = lane * kStride + (ts - t0) + i;
              wGB[li] = 0.0f;
              wDD[li] = 0.0f;
              if constexpr (kHasZ) wY[li] = 0.0f;
            }
          }
          continue;
        }
        float Av[4], A2v[4], Hc[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int n = G * 4 + s;
          const bool ok = ch_ok && n < N;
          Av[s] = ok ? Ap[(size_t)ch * N + n] : 0.0f;
          A2v[s] = Av[s] * kLog2e;
          float hc = 0.0f;
          if (ok) {
            if (c > 0) hc = h_chunks[((rb + ch) * p.nchunks + (c - 1)) * N + n];
            else if (h_init) hc = h_init[(rb + ch) * N + n];
          }
          Hc[s] = hc;
        }
        // recompute the 16 states and decays of the sub-chunk
        float a[4][kSub], H[4][kSub];
#pragma unroll
        for (int jq = 0; jq < kSub / 4; ++jq) {
          const int t4 = k * (kSub / 4) + jq;
          float dlv[4], duv[4];
          f4_to(sDelta[t4][lane], dlv);
          f4_to(sDu[t4][lane], duv);
          BC4 v;
          load_bc_block(bc, bc_offset(b, G, ngroups, Lp, ts + 4 * jq), v);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int i = 4 * jq + j;
            float yv = 0.0f;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
              a[s][i] = fast_exp2(dlv[j] * A2v[s]);
              const float hp = i ? H[s][i - 1] : Hc[s];
              H[s][i] = fmaf(a[s][i], hp, duv[j] * v.B(j, s));
              if constexpr (kHasZ) yv = fmaf(v.C(j, s), H[s][i], yv);
            }
            if constexpr (kHasZ) {
              float* dst = wY + lane * kStride + (ts - t0) + i;
              *dst = (g == 0) ? yv : *dst + yv;
            }
          }
        }
        // reverse recurrence
        float vals[2 * 4 * kSub];  // [kind: 0 dB, 1 dC][s][i]
#pragma unroll
        for (int jq = kSub / 4 - 1; jq >= 0; --jq) {
          const int t4 = k * (kSub / 4) + jq;
          float dlv[4], duv[4], dov[4];
          f4_to(sDelta[t4][lane], dlv);
          f4_to(sDu[t4][lane], duv);
          f4_to(sDout[t4][lane], dov);
          BC4 v;
          load_bc_block(bc, bc_offset(b, G, ngroups, Lp, ts + 4 * jq), v);
#pragma unroll
          for (int j = 3; j >= 0; --j) {
            const int i = 4 * jq + j;
            float gB = 0.0f, gD = 0.0f;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
              const float Gt = fmaf(dov[j], v.C(j, s), gam[g][s]);
              gB = fmaf(Gt, v.B(j, s), gB);
              const float hp = i ? H[s][i - 1] : Hc[s];
              const float gah = Gt * a[s][i] * hp;
              gD = fmaf(Av[s], gah, gD);
              dA[g][s] = fmaf(dlv[j], gah, dA[g][s]);
              vals[s * kSub + i] = Gt * duv[j];
              vals[4 * kSub + s * kSub + i] = dov[j] * H[s][i];
              gam[g][s] = a[s][i] * Gt;
            }
            const int li = lane * kStride + (ts - t0) + i;
            wGB[li] = (g == 0) ? gB : wGB[li] + gB;
            wDD[li] = (g == 0) ? gD : wDD[li] + gD;
          }
        }
        // sum over the 64 channels of this block: lane holds indices 2*lane, 2*lane+1
        wave_reduce_scatter<2 * 4 * kSub>(vals, lane);
        {
          const int kind = lane >> 5;
          const int s = (lane >> 3) & 3;
          const int i0 = (lane & 7) * 2;
          const int n = G * 4 + s;
          const int t = ts + i0;
          if (n < N) {
            float* dst = ws_bc + ((size_t)kind * p.nblk + blk) * nBC + ((size_t)b * N + n) * L;
            if (t < L) dst[t] = vals[0];
            if (t + 1 < L) dst[t + 1] = vals[1];
          }
        }
      }
    }
    __syncthreads();

    // ---- phase C: per-position gradients
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) {
      const int row = a_row + ps * kRPP;
      const int c = d0 + row;
      const int t = t0 + a_col;
      float duo[kVec], ddo[kVec], dzo[kVec];
#pragma unroll
      for (int q = 0; q < kVec / 4; ++q) {
        const int t4 = a_col / 4 + q;
        float de[4], uu[4], dov[4], xv[4];
        f4_to(sDelta[t4][row], de);
        f4_to(sU[t4][row], uu);
        f4_to(sDout[t4][row], dov);
        f4_to(sX[t4][row], xv);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int tl = a_col + 4 * q + j;
          const int li = row * kStride + tl;
          const float gb = (sGB[li] + sGB[kSlice + li]) + (sGB[2 * kSlice + li] + sGB[3 * kSlice + li]);
          const float gd = (sDD[li] + sDD[kSlice + li]) + (sDD[2 * kSlice + li] + sDD[3 * kSlice + li]);
          const int tt = t + 4 * q + j;
          const bool valid = tt >= vlo && tt < vhi;
          const float ddl = fmaf(uu[j], gb, gd);
          const float dsp = softplus ? softplus_grad_t20(xv[j]) : 1.0f;
          const float dd = valid ? ddl * dsp : 0.0f;
          duo[4 * q + j] = fmaf(Dv[ps], dov[j], de[j] * gb);
          ddo[4 * q + j] = dd;
          accD[ps] = fmaf(dov[j], uu[j], accD[ps]);
          accB[ps] += dd;
          if constexpr (kHasZ) {
            const float ys = (sY[li] + sY[kSlice + li]) + (sY[2 * kSlice + li] + sY[3 * kSlice + li]);
            const float yo = fmaf(Dv[ps], uu[j], ys);
            dzo[4 * q + j] = dzf[ps][4 * q + j] * yo;
          }
        }
      }
      if (c < Dm && t < L) {
        store_row<T, kAligned>(dup + (rb + c) * L, t, L, duo);
        store_row<T, kAligned>(ddp + (rb + c) * L, t, L, ddo);
        if constexpr (kHasZ) store_row<T, kAligned>(dzp + (rb + c) * L, t, L, dzo);
      }
    }
    // the next tile's phase B overwrites the slices only after the barrier
    // that ends its phase A, so no barrier is needed here
  }

  // ---- per-row partials
#pragma unroll
  for (int g = 0; g < kSG; ++g)
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int n = (g * kWaves + w) * 4 + s;
      if (ch_ok && n < N) {
        ws_A[(rb + ch) * N + n] = dA[g][s];
        if (dh_init) dh_init[(rb + ch) * N + n] = gam[g][s];
      }
    }
#pragma unroll
  for (int ps = 0; ps < kPasses; ++ps) {
    const float sd = group_sum<kLPR>(accD[ps]);
    const float sb = group_sum<kLPR>(accB[ps]);
    const int c = d0 + a_row + ps * kRPP;
    if ((tid % kLPR) == 0 && c < Dm) {
      ws_D[rb + c] = sd;
      ws_bias[rb + c] = sb;
    }
  }
}

// Adds the partial sums: dB/dC over channel blocks, dA/dD/dbias over batch rows.
template <typename T>
__global__ __launch_bounds__(256) void scan_bwd_reduce_kernel(
    const int batch, const int dim, const int N, const int L, const int nblk,
    const float* __restrict__ ws_bc, const float* __restrict__ ws_A,
    const float* __restrict__ ws_D, const float* __restrict__ ws_bias, T* __restrict__ dB,
    T* __restrict__ dC, float* __restrict__ dA, float* __restrict__ dD,
    float* __restrict__ dbias) {
  const size_t nBC = (size_t)batch * N * L;
  const size_t nA = (size_t)dim * N;
  const size_t total = 2 * nBC + nA + dim;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    if (i < 2 * nBC) {
      const size_t kind = i / nBC, r = i % nBC;
      const float* src = ws_bc + kind * nblk * nBC + r;
      float s = 0.0f;
      for (int k = 0; k < nblk; ++k) s += src[(size_t)k * nBC];
      Elem<T>::store1((kind ? dC : dB) + r, s);
    } else if (i < 2 * nBC + nA) {
      const size_t r = i - 2 * nBC;
      float s = 0.0f;
      for (int bb = 0; bb < batch; ++bb) s += ws_A[(size_t)bb * nA + r];
      dA[r] = s;
    } else {
      const size_t d = i - 2 * nBC - nA;
      float sd = 0.0f, sb = 0.0f;
      for (int bb = 0; bb < batch; ++bb) {
        sd += ws_D[(size_t)bb * dim + d];
        sb += ws_bias[(size_t)bb * dim + d];
      }
      if (dD) dD[d] = sd;
      if (dbias) dbias[d] = sb;
    }
  }
}

// ---------------------------------------------------------------- launch

size_t bc_prep_floats(int batch, int nstate, int seqlen);
hipError_t launch_bc_prep(const ScanParams& p, int dtype, float* bc, hipStream_t st);

size_t bwd_ws_floats(int batch, int dim, int nstate, int seqlen) {
  const size_t nblk = (dim + kBlockCh - 1) / kBlockCh;
  return 2 * nblk * (size_t)batch * nstate * seqlen   // dB/dC partials
         + (size_t)batch * dim * nstate              // dA partials
         + 2 * (size_t)batch * dim;                  // dD, dbias partials
}

template <typename T, int kSG, bool kHasZ, bool kAligned>
static hipError_t launch_bwd4(const ScanParams& p, const float* bc, hipStream_t st) {
  dim3 grid(p.nblk, p.batch);
  ProfScope prof("scan_bwd", st);
  hipLaunchKernelGGL((scan_bwd_kernel<T, kSG, kHasZ, kAligned>), grid, dim3(256), 0, st,
                     dims_of(p), (const T*)p.u, (const T*)p.delta, p.A, bc, p.D, p.bias,
                     p.h_init, p.length, (const T*)p.z, p.h_chunks_in, (const T*)p.dout,
                     p.dh_last, (T*)p.du, (T*)p.ddelta, (T*)p.dz, p.dh_init, p.ws_bc, p.ws_A,
                     p.ws_D, p.ws_bias);
  return hipGetLastError();
}

template <typename T, int kSG>
static hipError_t launch_bwd3(const ScanParams& p, const float* bc, bool aligned, hipStream_t st) {
  if (p.z)
    return aligned ? launch_bwd4<T, kSG, true, true>(p, bc, st)
                   : launch_bwd4<T, kSG, true, false>(p, bc, st);
  return aligned ? launch_bwd4<T, kSG, false, true>(p, bc, st)
                 : launch_bwd4<T, kSG, false, false>(p, bc, st);
}

template <typename T>
static hipError_t launch_bwd2(const ScanParams& p, const float* bc, bool aligned, hipStream_t st) {
  hipError_t e;
  if (p.nstate <= 16) e = launch_bwd3<T, 1>(p, bc, aligned, st);
  else if (p.nstate <= 32) e = launch_bwd3<T, 2>(p, bc, aligned, st);
  else e = launch_bwd3<T, 4>(p, bc, aligned, st);
  if (e != hipSuccess) return e;
  const size_t total = 2 * (size_t)p.batch * p.nstate * p.seqlen + (size_t)p.dim * p.nstate + p.dim;
  const int blocks = (int)std::min<size_t>((total + 255) / 256, 16384);
  ProfScope prof("scan_bwd_reduce", st);
  hipLaunchKernelGGL(scan_bwd_reduce_kernel<T>, dim3(blocks), dim3(256), 0, st, p.batch, p.dim,
                     p.nstate, p.seqlen, p.nblk, p.ws_bc, p.ws_A, p.ws_D, p.ws_bias, (T*)p.dB,
                     (T*)p.dC, p.dA, p.dD, p.dbias);
  return hipGetLastError();
}

// bc must hold bc_prep_floats() floats; ws_* must be laid out by the caller
// (see bwd_ws_floats).  nstate <= 64.
hipError_t launch_scan_bwd(const ScanParams& p, int dtype, bool aligned, float* bc,
                           hipStream_t st) {
  hipError_t e = launch_bc_prep(p, dtype, bc, st);
  if (e != hipSuccess) return e;
  if (dtype == 1) return launch_bwd2<__hip_bfloat16>(p, bc, aligned, st);
  return launch_bwd2<float>(p, bc, aligned, st);
}

}  // namespace ssm
