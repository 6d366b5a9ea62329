// Selective-scan forward for gfx950.
//
// Computes, per (b, d) row (reference semantics: csrc/selective_scan/
// forward_kernel.cu:136-243):
//   delta_t = softplus(delta_raw_t + bias_d)   (identity step when t is padded)
//   h_t     = exp(delta_t * A_dn) * h_{t-1} + delta_t * u_t * B_nt
//   out_t   = D_d * u_t + sum_n C_nt * h_t     (* silu(z_t) when z is given)
//
// Work decomposition (one workgroup = one batch row b x 64 channels, 4 waves):
//   phase A  all 256 threads stream a 64-channel x 64-step tile of u / delta
//            (/ z) with 128-bit coalesced loads, evaluate softplus once per
//            element and stage delta and delta*u in LDS as float4 columns;
//   phase B  lane = channel, wave w = state group G = g*4 + w (4 states each):
//            a sequential recurrence over the 64 steps held in registers.  B
//            and C are wave-uniform (same b, n, t across the wave) and come
//            from the prepped fp32 block layout through scalar loads, so they
//            cost no VALU or LDS bandwidth.  Each wave leaves its partial sum
//            over its states of C*h in LDS;
//   phase C  the same threads as phase A add the four partials, D*u and the
//            z gate, and store the tile with 128-bit stores.
// The state after every kChunk steps is saved for the backward (h_chunks).
#include "ss_io.cuh"
#include "ss_params.h"
#include "ss_prof.h"

namespace ssm {

// ---------------------------------------------------------------- B/C prep

// bc[b][G][t][s][0/1] = B/C[b][4G+s][t] as fp32 (zero for padded states/steps);
// rows are bc_row_len(L) steps long.
template <typename T>
__global__ __launch_bounds__(256) void bc_prep_kernel(const int batch, const int N, const int L,
                                                      const int ngroups, const int Lp,
                                                      const T* __restrict__ Bp,
                                                      const T* __restrict__ Cp,
                                                      float* __restrict__ bc) {
  const size_t total = (size_t)batch * ngroups * Lp;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const int t = (int)(i % Lp);
    const size_t bg = i / Lp;
    const int G = (int)(bg % ngroups);
    const int b = (int)(bg / ngroups);
    float v[8];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int n = G * 4 + s;
      const bool ok = n < N && t < L;
      const size_t src = ((size_t)b * N + n) * L + t;
      v[2 * s] = ok ? Elem<T>::load1(Bp + src) : 0.0f;
      v[2 * s + 1] = ok ? Elem<T>::load1(Cp + src) : 0.0f;
    }
    float4* dst = reinterpret_cast<float4*>(bc + i * 8);
    dst[0] = make_float4(v[0], v[1], v[2], v[3]);
    dst[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// ---------------------------------------------------------------- forward

// Every pointer is its own __restrict__ argument: with that no-alias
// information the compiler can prove the output stores never clobber the
// prepped B/C block, which is what lets its wave-uniform reads be scalar loads.
template <typename T, int kSG, bool kHasZ, bool kAligned>
__global__ __launch_bounds__(256) void scan_fwd_kernel(
    const ScanDims p, const T* __restrict__ u, const T* __restrict__ dl,
    const float* __restrict__ Ap, const float* __restrict__ bc,
    const float* __restrict__ Dp, const float* __restrict__ biasp,
    const float* __restrict__ h_init, const int64_t* __restrict__ length,
    const T* __restrict__ zp, T* __restrict__ out, float* __restrict__ h_chunks,
    float* __restrict__ h_last) {
  using E = Elem<T>;
  constexpr int kWaves = 4;
  constexpr int kThreads = 64 * kWaves;
  constexpr int kVec = E::kVec;
  constexpr int kLPR = kTileT / kVec;    // threads per channel row of a tile
  constexpr int kRPP = kThreads / kLPR;  // rows per pass
  constexpr int kPasses = kBlockCh / kRPP;
  constexpr int kT4 = kTileT / 4;

  __shared__ float4 sDelta[kT4][kBlockCh];
  __shared__ float4 sDu[kT4][kBlockCh];
  __shared__ float4 sY[kWaves][kT4][kBlockCh];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = wave_id_uniform();
  const int b = blockIdx.y;
  const int d0 = blockIdx.x * kBlockCh;
  const int L = p.seqlen, Dm = p.dim, N = p.nstate;
  const int ngroups = (N + 3) / 4;
  const int Lp = bc_row_len(L);
  const size_t rb = (size_t)b * Dm;

  int vlo, vhi;
  valid_window(length, p.pad_right, b, L, vlo, vhi);

  // ---- scan lane state
  const int ch = d0 + lane;
  const bool ch_ok = ch < Dm;
  float h[kSG][4], A2[kSG][4];
#pragma unroll
  for (int g = 0; g < kSG; ++g)
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int n = (g * kWaves + w) * 4 + s;
      const bool ok = ch_ok && n < N;
      A2[g][s] = ok ? Ap[(size_t)ch * N + n] * kLog2e : 0.0f;
      h[g][s] = (ok && h_init) ? h_init[(rb + ch) * N + n] : 0.0f;
    }

  // ---- tile-phase mapping
  const int a_row = tid / kLPR;
  const int a_col = (tid % kLPR) * kVec;
  float Dv[kPasses], Bias[kPasses];
#pragma unroll
  for (int ps = 0; ps < kPasses; ++ps) {
    const int c = d0 + a_row + ps * kRPP;
    Dv[ps] = (c < Dm && Dp) ? Dp[c] : 0.0f;
    Bias[ps] = (c < Dm && biasp) ? biasp[c] : 0.0f;
  }
  const bool softplus = p.softplus != 0;
  const bool save = h_chunks != nullptr;

  for (int t0 = 0; t0 < L; t0 += kTileT) {
    // ---- phase A
    float uv[kPasses][kVec];
    float zv[kHasZ ? kPasses : 1][kVec];
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) {
      const int row = a_row + ps * kRPP;
      const int c = d0 + row;
      const int t = t0 + a_col;
      const bool ok = c < Dm;
      float dv[kVec];
      load_row<T, kAligned>(u + (rb + c) * L, t, L, ok, uv[ps]);
      load_row<T, kAligned>(dl + (rb + c) * L, t, L, ok, dv);
      if constexpr (kHasZ) load_row<T, kAligned>(zp + (rb + c) * L, t, L, ok, zv[ps]);
      float de[kVec], du[kVec];
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        const float x = dv[j] + Bias[ps];
        const float dt = softplus ? softplus_t20(x) : x;
        const int tt = t + j;
        const bool valid = tt >= vlo && tt < vhi;
        de[j] = valid ? dt : 0.0f;
        du[j] = de[j] * uv[ps][j];
      }
#pragma unroll
      for (int q = 0; q < kVec / 4; ++q) {
        sDelta[a_col / 4 + q][row] = make_float4(de[4 * q], de[4 * q + 1], de[4 * q + 2], de[4 * q + 3]);
        sDu[a_col / 4 + q][row] = make_float4(du[4 * q], du[4 * q + 1], du[4 * q + 2], du[4 * q + 3]);
      }
    }
    __syncthreads();

    // ---- phase B
    const int nT4 = min(kT4, (L - t0 + 3) / 4);
    for (int t4 = 0; t4 < nT4; ++t4) {
      float dlv[4], duv[4];
      f4_to(sDelta[t4][lane], dlv);
      f4_to(sDu[t4][lane], duv);
      float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      const int tb = t0 + 4 * t4;
#pragma unroll
      for (int g = 0; g < kSG; ++g) {
        const int G = g * kWaves + w;
        if (G < ngroups) {
          BC4 v;
          load_bc_block(bc, bc_offset(b, G, ngroups, Lp, tb), v);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int s = 0; s < 4; ++s) {
              const float a = fast_exp2(dlv[j] * A2[g][s]);
              h[g][s] = fmaf(a, h[g][s], duv[j] * v.B(j, s));
              y[j] = fmaf(v.C(j, s), h[g][s], y[j]);
            }
          }
        }
      }
      sY[w][t4][lane] = make_float4(y[0], y[1], y[2], y[3]);
      if (save && (((t4 & 3) == 3) || t4 == nT4 - 1) && ch_ok) {
        const int c = tb / kChunk;
        float* hc = h_chunks + ((rb + ch) * p.nchunks + c) * N;
#pragma unroll
        for (int g = 0; g < kSG; ++g)
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const int n = (g * kWaves + w) * 4 + s;
            if (n < N) hc[n] = h[g][s];
          }
      }
    }
    __syncthreads();

    // ---- phase C
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) {
      const int row = a_row + ps * kRPP;
      const int c = d0 + row;
      const int t = t0 + a_col;
      if (c < Dm && t < L) {
        float y[kVec];
#pragma unroll
        for (int q = 0; q < kVec / 4; ++q) {
          const float4 y0 = sY[0][a_col / 4 + q][row];
          const float4 y1 = sY[1][a_col / 4 + q][row];
          const float4 y2 = sY[2][a_col / 4 + q][row];
          const float4 y3 = sY[3][a_col / 4 + q][row];
          y[4 * q + 0] = (y0.x + y1.x) + (y2.x + y3.x);
          y[4 * q + 1] = (y0.y + y1.y) + (y2.y + y3.y);
          y[4 * q + 2] = (y0.z + y1.z) + (y2.z + y3.z);
          y[4 * q + 3] = (y0.w + y1.w) + (y2.w + y3.w);
        }
#pragma unroll
        for (int j = 0; j < kVec; ++j) {
          float v = fmaf(Dv[ps], uv[ps][j], y[j]);
          if constexpr (kHasZ) v *= silu_f(zv[ps][j]);
          y[j] = v;
        }
        store_row<T, kAligned>(out + (rb + c) * L, t, L, y);
      }
    }
  }

  if (!save && h_last && ch_ok) {
#pragma unroll
    for (int g = 0; g < kSG; ++g)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int n = (g * kWaves + w) * 4 + s;
        if (n < N) h_last[(rb + ch) * N + n] = h[g][s];
      }
  }
}

// ---------------------------------------------------------------- launch

size_t bc_prep_floats(int batch, int nstate, int seqlen) {
  const size_t ngroups = (nstate + 3) / 4;
  return (size_t)batch * ngroups * bc_row_len(seqlen) * 8;
}

hipError_t launch_bc_prep(const ScanParams& p, int dtype, float* bc, hipStream_t st) {
  const int ngroups = (p.nstate + 3) / 4;
  const int Lp = bc_row_len(p.seqlen);
  const size_t total = (size_t)p.batch * ngroups * Lp;
  const int blocks = (int)std::min<size_t>((total + 255) / 256, 65535);
  ProfScope prof("bc_prep", st);
  if (dtype == 1)
    hipLaunchKernelGGL(bc_prep_kernel<__hip_bfloat16>, dim3(blocks), dim3(256), 0, st, p.batch,
                       p.nstate, p.seqlen, ngroups, Lp, (const __hip_bfloat16*)p.B,
                       (const __hip_bfloat16*)p.C, bc);
  else
    hipLaunchKernelGGL(bc_prep_kernel<float>, dim3(blocks), dim3(256), 0, st, p.batch, p.nstate,
                       p.seqlen, ngroups, Lp, (const float*)p.B, (const float*)p.C, bc);
  return hipGetLastError();
}

template <typename T, int kSG, bool kHasZ, bool kAligned>
static hipError_t launch_fwd4(const ScanParams& p, const float* bc, hipStream_t st) {
  dim3 grid(p.nblk, p.batch);
  ProfScope prof("scan_fwd", st);
  hipLaunchKernelGGL((scan_fwd_kernel<T, kSG, kHasZ, kAligned>), grid, dim3(256), 0, st,
                     dims_of(p), (const T*)p.u, (const T*)p.delta, p.A, bc, p.D, p.bias,
                     p.h_init, p.length, (const T*)p.z, (T*)p.out, p.h_chunks, p.h_last);
  return hipGetLastError();
}

template <typename T, int kSG>
static hipError_t launch_fwd3(const ScanParams& p, const float* bc, bool aligned, hipStream_t st) {
  const bool z = p.z != nullptr;
  if (z)
    return aligned ? launch_fwd4<T, kSG, true, true>(p, bc, st)
                   : launch_fwd4<T, kSG, true, false>(p, bc, st);
  return aligned ? launch_fwd4<T, kSG, false, true>(p, bc, st)
                 : launch_fwd4<T, kSG, false, false>(p, bc, st);
}

template <typename T>
static hipError_t launch_fwd2(const ScanParams& p, const float* bc, bool aligned, hipStream_t st) {
  if (p.nstate <= 16) return launch_fwd3<T, 1>(p, bc, aligned, st);
  if (p.nstate <= 32) return launch_fwd3<T, 2>(p, bc, aligned, st);
  if (p.nstate <= 64) return launch_fwd3<T, 4>(p, bc, aligned, st);
  return launch_fwd3<T, 16>(p, bc, aligned, st);
}

// bc must hold bc_prep_floats() floats; it is filled here before the scan.
hipError_t launch_scan_fwd(const ScanParams& p, int dtype, bool aligned, float* bc,
                           hipStream_t st) {
  hipError_t e = launch_bc_prep(p, dtype, bc, st);
  if (e != hipSuccess) return e;
  if (dtype == 1) return launch_fwd2<__hip_bfloat16>(p, bc, aligned, st);
  return launch_fwd2<float>(p, bc, aligned, st);
}

}  // namespace ssm
