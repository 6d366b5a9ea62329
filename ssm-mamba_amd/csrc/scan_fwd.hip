// Selective-scan forward for gfx950.
//
// Computes, per (b, d) row (reference semantics: csrc/selective_scan/
// forward_kernel.cu:136-243):
//   delta_t = softplus(delta_raw_t + bias_d)   (identity step when t is padded)
//   h_t     = exp(delta_t * A_dn) * h_{t-1} + delta_t * u_t * B_nt
//   out_t   = D_d * u_t + sum_n C_nt * h_t     (* silu(z_t) when z is given)
//
// Work decomposition (one workgroup = one batch row b x 64 channels, 8 waves,
// two waves per SIMD):
//   phase A  the 512 threads stream a 64-channel x 32-step tile of u / delta
//            (/ z) (4 consecutive steps per thread, coalesced rows), evaluate
//            softplus once per element and stage delta and delta*u in LDS as
//            float4 columns.  The next tile's rows are already in flight: they
//            are loaded during the previous tile's phase B;
//   phase B  lane = channel, wave w = state pairs G = g*8 + w: a sequential
//            recurrence over the tile held in registers.  B and C are
//            wave-uniform (same b, n, t across the wave).  With N <= 16 phase A
//            reads them straight from B and C (coalesced along the steps) and
//            stages the super-tile's (B0, C0, B1, C1) per pair and step in LDS,
//            read back with broadcast loads; larger N read the prepped fp32
//            block layout through scalar loads.  Each 4-step block's loads are
//            issued one block ahead.  Each wave leaves its partial sum over its
//            states of C*h in its own LDS slice;
//   phase C  the phase-A threads add the eight slices in a fixed order, D*u
//            and the z gate, and store the tile.
// The state after every kChunk steps is saved for the backward (h_chunks,
// laid out (batch, nchunks, nstate, dim) so the saves are coalesced).
#include "ss_io.cuh"
#include "ss_params.h"
#include "ss_prof.h"

namespace ssm {

// ---------------------------------------------------------------- B/C prep

// bc[b][G][t][s][0/1] = B/C[b][2G+s][t] as fp32 (zero for padded states and
// steps); rows are bc_row_len(L) steps long.
template <typename T>
__global__ __launch_bounds__(256) void bc_prep_kernel(const int batch, const int N, const int L,
                                                      const int npair, const int Lp,
                                                      const T* __restrict__ Bp,
                                                      const T* __restrict__ Cp,
                                                      const int64_t bstride,
                                                      float* __restrict__ bc) {
  const size_t total = (size_t)batch * npair * Lp;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const int t = (int)(i % Lp);
    const size_t bg = i / Lp;
    const int G = (int)(bg % npair);
    const int b = (int)(bg / npair);
    float v[4];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int n = G * 2 + s;
      const bool ok = n < N && t < L;
      const size_t src = (size_t)b * bstride + (size_t)n * L + t;
      v[2 * s] = ok ? Elem<T>::load1(Bp + src) : 0.0f;
      v[2 * s + 1] = ok ? Elem<T>::load1(Cp + src) : 0.0f;
    }
    reinterpret_cast<float4*>(bc)[i] = make_float4(v[0], v[1], v[2], v[3]);
  }
}

// ---------------------------------------------------------------- forward

// LDS column swizzle.  Tile columns (4-step groups q = 0..7) of 64 channel
// rows are stored at row index r ^ col_swz(q).  Phase A/C threads access one
// row's 8 columns across 8 consecutive lanes, and without the swizzle those
// columns (1 KiB apart) fall in the same banks; with it every 8- or 16-lane
// group of a ds_write_b128 / ds_read_b128 touches distinct banks.  Phase B
// reads whole columns, a permutation of 64 consecutive float4s.
__device__ __forceinline__ constexpr int col_swz(int q) { return q | ((q & 1) << 3); }

// A 4-step block of one state pair's prepped B/C from LDS (the same address
// in every lane: broadcast reads).
__device__ __forceinline__ void lds_bc_block(const float4* __restrict__ row, int step, BC2& r) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float4 q = row[step + j];
    r.v[4 * j] = q.x; r.v[4 * j + 1] = q.y; r.v[4 * j + 2] = q.z; r.v[4 * j + 3] = q.w;
  }
}

// One 4-step block of the recurrence for the wave's 2 states.
__device__ __forceinline__ void fwd_block(const float4 dl4, const float4 du4, const BC2& v,
                                          const float (&A2)[2], float (&h)[2], float (&y)[4]) {
  const float dlv[4] = {dl4.x, dl4.y, dl4.z, dl4.w};
  const float duv[4] = {du4.x, du4.y, du4.z, du4.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const float a = fast_exp2(dlv[j] * A2[s]);
      h[s] = fmaf(a, h[s], duv[j] * v.B(j, s));
      y[j] = fmaf(v.C(j, s), h[s], y[j]);
    }
  }
}

// The same block without outputs (the segment summaries).
__device__ __forceinline__ void fwd_block_state(const float4 dl4, const float4 du4, const BC2& v,
                                                const float (&A2)[2], float (&h)[2]) {
  const float dlv[4] = {dl4.x, dl4.y, dl4.z, dl4.w};
  const float duv[4] = {du4.x, du4.y, du4.z, du4.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int s = 0; s < 2; ++s) h[s] = fmaf(fast_exp2(dlv[j] * A2[s]), h[s], duv[j] * v.B(j, s));
  }
}

// Every pointer is its own __restrict__ argument: with that no-alias
// information the compiler can prove the output stores never clobber the
// prepped B/C block, which is what lets its wave-uniform reads be scalar loads.
//
// Sequence split (p.nseg > 1, blockIdx.z = segment s of p.seg_len steps):
// segment s starts from h_init folded through the summaries of segments
// 0..s-1 left by scan_fwd_segsum_kernel (h <- exp(A sum dt) h + h_seg, the
// composition of the steps' affine maps).
//
// kZ: 0 no gate; 1 out = y * silu(z); 2 the same and the ungated y also
// written to yu (the value the backward needs for dz).
template <typename T, int kSG, int kZ, bool kAligned>
__global__ __launch_bounds__(kThreads) void scan_fwd_kernel(
    const ScanDims p, const T* __restrict__ u, const T* __restrict__ dl,
    const float* __restrict__ Ap, const float* __restrict__ bc, const T* __restrict__ Bp,
    const T* __restrict__ Cp, const float* __restrict__ Dp, const float* __restrict__ biasp,
    const float* __restrict__ h_init, const int64_t* __restrict__ length,
    const T* __restrict__ zp, T* __restrict__ out, T* __restrict__ yu,
    float* __restrict__ h_chunks, float* __restrict__ h_last, void* __restrict__ dummy,
    const float* __restrict__ seg_h, const float* __restrict__ seg_dt) {
  using R4 = typename Raw4<T>::type;
  constexpr bool kHasZ = kZ != 0;
  constexpr bool kSaveY = kZ == 2;
  constexpr int kT4 = kTileF / 4;        // 4-step columns per sub-tile
  constexpr int kSup = kSubF * kTileF;   // steps staged per super-tile
  static_assert(kBlockCh * kT4 == kThreads, "one 4-step row piece per thread");

  __shared__ float4 sDelta[kSubF * kT4][kBlockCh];
  __shared__ float4 sDu[kSubF * kT4][kBlockCh];
  __shared__ float4 sY[kWaves][kT4][kBlockCh];
  // prepped B/C of the super-tile for state pairs 0..7: [sub][pair][step]
  __shared__ float4 sBC[kSubF][kWaves][kTileF];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = wave_id_uniform();
  const int b = blockIdx.y;
  const int d0 = blockIdx.x * kBlockCh;
  const int L = p.seqlen, Dm = p.dim, N = p.nstate;
  // this workgroup's steps [Tbeg, Lend); rows are still addressed with L
  const int seg = blockIdx.z;
  const int Tbeg = seg * p.seg_len;
  const int Lend = min(L, Tbeg + p.seg_len);
  const int ngroups = (N + 1) / 2;
  const int npair = bc_pairs(N);
  const int Lp = bc_row_len(L);
  const size_t rb = (size_t)b * Dm;

  int vlo, vhi;
  valid_window(length, p.pad_right, b, L, vlo, vhi);

  // ---- scan lane state
  const int ch = d0 + lane;
  const bool ch_ok = ch < Dm;
  float h[kSG][2], A2[kSG][2];
#pragma unroll
  for (int g = 0; g < kSG; ++g)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int n = (g * kWaves + w) * 2 + s;
      const bool ok = ch_ok && n < N;
      A2[g][s] = ok ? Ap[(size_t)ch * N + n] * kLog2e : 0.0f;
      float hv = (ok && h_init) ? h_init[(rb + ch) * N + n] : 0.0f;
      // carry in through the earlier summaries' affine maps, in order
      if (ok)
        hv = fold_carry(hv, A2[g][s], seg_dt, seg_h, 0, 1, seg * p.sub_k, p.batch, b, Dm, N, n, ch);
      h[g][s] = hv;
    }

  // ---- tile-phase mapping: thread = (channel row, 4 consecutive steps of
  // every sub-tile)
  const int a_row = tid / kT4;
  const int a_q = tid % kT4;
  const int a_col = a_q * 4;
  const int a_sw = a_row ^ col_swz(a_q);
  const int a_ch = d0 + a_row;
  const bool a_ok = a_ch < Dm;
  const float Dv = (a_ok && Dp) ? Dp[a_ch] : 0.0f;
  const float Bias = (a_ok && biasp) ? biasp[a_ch] : 0.0f;
  // rows of the clamped channel (always valid addresses; loads of rows past
  // the last channel are zeroed)
  const int a_chc = min(a_ch, Dm - 1);
  const T* __restrict__ u_row = u + (rb + a_chc) * L;
  const T* __restrict__ d_row = dl + (rb + a_chc) * L;
  const T* __restrict__ z_row = zp + (rb + a_chc) * L;
  const bool softplus = p.softplus != 0;
  const bool save = h_chunks != nullptr;
  const size_t hsD = (size_t)p.hs * Dm;  // floats between the saved rows of two states
  float* const dummyf = static_cast<float*>(dummy);

  // Raw row pieces of the next super-tile, all loads issued at once right
  // after the current super-tile's phase A.  They are consumed together at
  // the next phase A, so each register is carried exactly one iteration.
  // Past the end the last sub-tile is re-read (unconditional loads keep the
  // registers free of merges).
  const int last_t0 = (Lend - 1) / kTileF * kTileF;
  R4 qu[kSubF], qd[kSubF], qz[kSubF];
  // B/C staging (kSG == 1): thread -> (pair, step) of the super-tile,
  // kBCPer items of (B0, C0, B1, C1) read straight from B and C (the states
  // 2G, 2G+1 of the pair; masked to zero at staging for states past N, so
  // those waves run the common path and add nothing)
  constexpr int kBCItems = kSubF * kWaves * kTileF;
  constexpr int kBCPer = kBCItems / kThreads;
  static_assert(kBCItems % kThreads == 0, "whole B/C items per thread");
  const T* __restrict__ Braw = static_cast<const T*>(Bp) + (size_t)b * p.bc_bstride;
  const T* __restrict__ Craw = static_cast<const T*>(Cp) + (size_t)b * p.bc_bstride;
  float qbc[kBCPer][4];
  auto issue = [&](int T0) {
#pragma unroll
    for (int i = 0; i < kSubF; ++i) {
      const int t = min(T0 + i * kTileF, last_t0) + a_col;
      qu[i] = load_raw4_nb<T, kAligned>(u_row, t, L, a_ok);
      qd[i] = load_raw4_nb<T, kAligned>(d_row, t, L, a_ok);
      if constexpr (kHasZ) qz[i] = load_raw4_nb<T, kAligned>(z_row, t, L, a_ok);
      else qz[i] = R4{};
    }
    if constexpr (kSG == 1) {
#pragma unroll
      for (int r = 0; r < kBCPer; ++r) {
        const int item = r * kThreads + tid;
        const int step = item % kTileF;
        const int G = (item / kTileF) % kWaves;
        const int sub = item / (kTileF * kWaves);
        // clamped into the rows (steps past L only meet delta = 0 and are
        // never stored; states past N are zeroed at staging)
        const int t = min(min(T0, last_t0) + sub * kTileF + step, L - 1);
        const size_t o0 = (size_t)min(2 * G, N - 1) * L + t;
        const size_t o1 = (size_t)min(2 * G + 1, N - 1) * L + t;
        qbc[r][0] = Elem<T>::load1(Braw + o0);
        qbc[r][1] = Elem<T>::load1(Craw + o0);
        qbc[r][2] = Elem<T>::load1(Braw + o1);
        qbc[r][3] = Elem<T>::load1(Craw + o1);
      }
    }
  };

  // kFull (whole super-tile inside the sequence, kSG == 1): the steady
  // state, with no branches around memory operations, so the compiler's
  // waits for the prefetched rows count exactly what is needed.  Otherwise
  // the general code (last super-tile, N > 16).
  //
  // The loop is rotated: a super-tile's phase A runs at the end of the
  // previous iteration, so the wait for its rows sits in the same iteration
  // as their loads and the stores issued after them (no loop-header merge in
  // between that would make the compiler wait for those stores too).
  float skip[kSubF][4], gate[kSubF][4];  // phase A -> phase C: D*u, silu(z)
  // ---- phase A: softplus once per element, stage delta and delta*u for
  // the whole super-tile; D*u and silu(z) are kept for phase C.
  auto phase_a = [&](const int T0, auto full_tag) {
    constexpr bool kFull = decltype(full_tag)::value;
#pragma unroll
    for (int i = 0; i < kSubF; ++i) {
      const int t0 = T0 + i * kTileF;
      if (kFull || t0 < Lend) {
        float uv[4], dv[4], de[4], du[4];
        decode4(qu[i], uv);
        decode4(qd[i], dv);
        if constexpr (kHasZ) {
          float zv[4];
          decode4(qz[i], zv);
#pragma unroll
          for (int j = 0; j < 4; ++j) gate[i][j] = silu_f(zv[j]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          skip[i][j] = Dv * uv[j];
          const float x = dv[j] + Bias;
          const float dt = softplus ? softplus_t20(x) : x;
          const int tt = t0 + a_col + j;
          const bool valid = a_ok && tt >= vlo && tt < vhi;
          de[j] = valid ? dt : 0.0f;
          du[j] = de[j] * uv[j];
        }
        sDelta[i * kT4 + a_q][a_sw] = make_float4(de[0], de[1], de[2], de[3]);
        sDu[i * kT4 + a_q][a_sw] = make_float4(du[0], du[1], du[2], du[3]);
      }
    }
    if constexpr (kSG == 1) {
#pragma unroll
      for (int r = 0; r < kBCPer; ++r) {
        const int item = r * kThreads + tid;
        const int G = (item / kTileF) % kWaves;
        const bool ok0 = 2 * G < N, ok1 = 2 * G + 1 < N;
        sBC[item / (kTileF * kWaves)][G][item % kTileF] =
            make_float4(ok0 ? qbc[r][0] : 0.0f, ok0 ? qbc[r][1] : 0.0f, ok1 ? qbc[r][2] : 0.0f,
                        ok1 ? qbc[r][3] : 0.0f);
      }
    }
  };

  // ---- phases B and C of the super-tile staged by the last phase A
  auto body = [&](const int T0, auto full_tag) {
    constexpr bool kFull = decltype(full_tag)::value;
    __syncthreads();
    issue(T0 + kSup);

#pragma unroll
    for (int i = 0; i < kSubF; ++i) {
      const int t0 = T0 + i * kTileF;
      if (!kFull && t0 >= Lend) break;
      const float4* __restrict__ cDelta = sDelta[i * kT4];
      const float4* __restrict__ cDu = sDu[i * kT4];
      // ---- phase B over sub-tile i
      const int nT4 = min(kT4, (Lend - t0 + 3) / 4);
      auto store_carry = [&](int t4) {
        if (save && (((t4 & 3) == 3) || t4 == nT4 - 1) && ch_ok) {
          // layout (batch, nchunks, nstate, dim): each state is one
          // contiguous 256 B run of the wave's 64 channels
          const int c = (t0 + 4 * t4) / kChunk;
          float* hc = h_chunks + ((size_t)b * p.nchunks + c) * N * hsD + ch;
#pragma unroll
          for (int g = 0; g < kSG; ++g)
#pragma unroll
            for (int s = 0; s < 2; ++s) {
              const int n = (g * kWaves + w) * 2 + s;
              if (n < N) hc[(size_t)n * hsD] = h[g][s];
            }
        }
      };
      if constexpr (kFull) {
        // every wave: full sub-tile, fully unrolled, static B/C offsets and
        // buffers; carries after blocks 3 and 7 (masked-off ones go to the
        // dummy slot).  Block k+1's LDS loads are issued right after block
        // k's have arrived, then block k is computed.
        const float4* __restrict__ cBC = sBC[i][w];
        const bool hc_ok = save && ch_ok && w < ngroups;
        const bool hc2_ok = hc_ok && 2 * w + 1 < N;
        float* const hc = h_chunks + (((size_t)b * p.nchunks + t0 / kChunk) * N + 2 * w) * hsD + ch;
        BC2 bcb[2];
        float4 dlb[2], dub[2];
        lds_bc_block(cBC, 0, bcb[0]);
        dlb[0] = cDelta[lane ^ col_swz(0)];
        dub[0] = cDu[lane ^ col_swz(0)];
#pragma unroll
        for (int k = 0; k < kT4; ++k) {
          const int c = k & 1;
          if (k + 1 < kT4) {
            dlb[c ^ 1] = cDelta[(k + 1) * kBlockCh + (lane ^ col_swz(k + 1))];
            dub[c ^ 1] = cDu[(k + 1) * kBlockCh + (lane ^ col_swz(k + 1))];
            lds_bc_block(cBC, 4 * (k + 1), bcb[c ^ 1]);
          }
          float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
          fwd_block(dlb[c], dub[c], bcb[c], A2[0], h[0], y);
          sY[w][k][lane ^ col_swz(k)] = make_float4(y[0], y[1], y[2], y[3]);
          if ((k & 3) == 3) {
            const size_t off = (size_t)(k / 4) * N * hsD;
            *(hc_ok ? hc + off : dummyf) = h[0][0];
            *(hc2_ok ? hc + off + hsD : dummyf) = h[0][1];
          }
        }
      } else if constexpr (kSG == 1) {
        if (w < ngroups && nT4 == kT4) {
          // full sub-tile, fully unrolled: static B/C offsets and buffers,
          // carries after blocks 3 and 7.  Block k+1's LDS and scalar loads
          // are issued right after block k's have arrived, then block k is
          // computed.
          const float4* __restrict__ cBC = sBC[i][w];
          float* hc = (save && ch_ok)
                          ? h_chunks + (((size_t)b * p.nchunks + t0 / kChunk) * N + 2 * w) * hsD + ch
                          : nullptr;
          const bool second = 2 * w + 1 < N;
          BC2 bcb[2];
          float4 dlb[2], dub[2];
          lds_bc_block(cBC, 0, bcb[0]);
          dlb[0] = cDelta[lane ^ col_swz(0)];
          dub[0] = cDu[lane ^ col_swz(0)];
#pragma unroll
          for (int k = 0; k < kT4; ++k) {
            const int c = k & 1;
            if (k + 1 < kT4) {
              dlb[c ^ 1] = cDelta[(k + 1) * kBlockCh + (lane ^ col_swz(k + 1))];
              dub[c ^ 1] = cDu[(k + 1) * kBlockCh + (lane ^ col_swz(k + 1))];
              lds_bc_block(cBC, 4 * (k + 1), bcb[c ^ 1]);
            }
            float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            fwd_block(dlb[c], dub[c], bcb[c], A2[0], h[0], y);
            sY[w][k][lane ^ col_swz(k)] = make_float4(y[0], y[1], y[2], y[3]);
            if ((k & 3) == 3 && hc) {
              float* q = hc + (size_t)(k / 4) * N * hsD;
              q[0] = h[0][0];
              if (second) q[hsD] = h[0][1];
            }
          }
        } else if (w < ngroups) {
          // partial last sub-tile: pairs of blocks; every prefetch is
          // unconditional (the index is clamped to the last block) so the
          // buffers stay in scalar registers
          const float4* __restrict__ cBC = sBC[i][w];
          float4 dlA = cDelta[lane ^ col_swz(0)], duA = cDu[lane ^ col_swz(0)], dlB, duB;
          BC2 bcA, bcB;
          lds_bc_block(cBC, 0, bcA);
          int t4 = 0;
          for (; t4 + 1 < nT4; t4 += 2) {
            dlB = cDelta[(t4 + 1) * kBlockCh + (lane ^ col_swz(t4 + 1))];
            duB = cDu[(t4 + 1) * kBlockCh + (lane ^ col_swz(t4 + 1))];
            lds_bc_block(cBC, 4 * (t4 + 1), bcB);
            {
              float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
              fwd_block(dlA, duA, bcA, A2[0], h[0], y);
              sY[w][t4][lane ^ col_swz(t4)] = make_float4(y[0], y[1], y[2], y[3]);
              store_carry(t4);
            }
            const int n2 = min(t4 + 2, nT4 - 1);
            dlA = cDelta[n2 * kBlockCh + (lane ^ col_swz(n2))];
            duA = cDu[n2 * kBlockCh + (lane ^ col_swz(n2))];
            lds_bc_block(cBC, 4 * n2, bcA);
            {
              float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
              fwd_block(dlB, duB, bcB, A2[0], h[0], y);
              sY[w][t4 + 1][lane ^ col_swz(t4 + 1)] = make_float4(y[0], y[1], y[2], y[3]);
              store_carry(t4 + 1);
            }
          }
          if (t4 < nT4) {  // odd last block
            float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            fwd_block(dlA, duA, bcA, A2[0], h[0], y);
            sY[w][t4][lane ^ col_swz(t4)] = make_float4(y[0], y[1], y[2], y[3]);
            store_carry(t4);
          }
        } else {
          for (int t4 = 0; t4 < nT4; ++t4) sY[w][t4][lane] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
      } else {
        for (int t4 = 0; t4 < nT4; ++t4) {
          const float4 dl4 = cDelta[t4 * kBlockCh + (lane ^ col_swz(t4))];
          const float4 du4 = cDu[t4 * kBlockCh + (lane ^ col_swz(t4))];
          float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
          const int tb = t0 + 4 * t4;
#pragma unroll
          for (int g = 0; g < kSG; ++g) {
            const int G = g * kWaves + w;
            if (G < ngroups) {
              BC2 v;
              load_bc_block(bc, bc_offset(b, G, npair, Lp, tb), v);
              fwd_block(dl4, du4, v, A2[g], h[g], y);
            }
          }
          sY[w][t4][lane ^ col_swz(t4)] = make_float4(y[0], y[1], y[2], y[3]);
          store_carry(t4);
        }
      }
      __syncthreads();

      // ---- phase C over sub-tile i: add the eight slices in a fixed order,
      // D*u and the gate
      {
        const int t = t0 + a_col;
        if (kFull || (a_ok && t < Lend)) {
          float y[4];
          float4 acc = sY[0][a_q][a_sw];
#pragma unroll
          for (int ww = 1; ww < kWaves; ++ww) {
            const float4 v = sY[ww][a_q][a_sw];
            acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
          }
          y[0] = skip[i][0] + acc.x;
          y[1] = skip[i][1] + acc.y;
          y[2] = skip[i][2] + acc.z;
          y[3] = skip[i][3] + acc.w;
          if constexpr (kSaveY) {
            if constexpr (kFull) store4_nb<T, kAligned>(yu + (rb + a_ch) * L, t, L, a_ok, dummy, y);
            else store4<T, kAligned>(yu + (rb + a_ch) * L, t, L, y);
          }
          if constexpr (kHasZ) {
#pragma unroll
            for (int j = 0; j < 4; ++j) y[j] *= gate[i][j];
          }
          if constexpr (kFull) store4_nb<T, kAligned>(out + (rb + a_ch) * L, t, L, a_ok, dummy, y);
          else store4<T, kAligned>(out + (rb + a_ch) * L, t, L, y);
        }
      }
      // the next sub-tile's phase B rewrites the slices
      if (i + 1 < kSubF && (kFull || t0 + kTileF < Lend)) __syncthreads();
    }
    // the next phase A rewrites only sDelta / sDu / sBC, last read by the
    // final phase B before the barrier that preceded the final phase C
  };

  issue(Tbeg);
  if (kSG == 1 && Tbeg + kSup <= Lend) phase_a(Tbeg, std::true_type{});
  else phase_a(Tbeg, std::false_type{});
  int T0 = Tbeg;
  if constexpr (kSG == 1) {
    for (; T0 + kSup <= Lend; T0 += kSup) {
      body(T0, std::true_type{});
      const int Tn = T0 + kSup;
      if (Tn + kSup <= Lend) phase_a(Tn, std::true_type{});
      else if (Tn < Lend) phase_a(Tn, std::false_type{});
    }
  }
  for (; T0 < Lend; T0 += kSup) {
    body(T0, std::false_type{});
    if (T0 + kSup < Lend) phase_a(T0 + kSup, std::false_type{});
  }

  if (!save && h_last && ch_ok && Lend == L) {
#pragma unroll
    for (int g = 0; g < kSG; ++g)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int n = (g * kWaves + w) * 2 + s;
        if (n < N) h_last[(rb + ch) * N + n] = h[g][s];
      }
  }
}

// ---------------------------------------------------------------- forward, N <= 16

// Role-split forward for up to 16 states.  A workgroup of 12 waves covers one
// batch row b x 64 channels and walks its segment in 16-step tiles (one saved
// chunk each):
//   consumer waves 0..7   lane = channel, wave w = states 2w and 2w+1: the
//                         recurrence over tile i, reading delta, delta*u and
//                         B/C from LDS; each wave leaves its partial sums of
//                         C*h in its own LDS slice;
//   producer waves 8..11  lane -> (channel row, 4-step column): stage tile
//                         i+2 (softplus, delta*u, B and C) and finish tile i-1
//                         (the eight slices added in a fixed order, D*u, the z
//                         gate, the stores; on the aligned path the outputs of
//                         four tiles are gathered in LDS and stored as whole
//                         64-step row pieces).
// Both roles run at the same time with one barrier per tile, so the
// producers' transcendental, conversion and store work fills the issue slots
// the recurrence leaves (a SIMD runs two consumer waves and one producer
// wave).  Staging runs two tiles ahead (three LDS buffers), so a tile's data
// is complete one barrier before it is needed: a consumer reads the first
// block of tile i+1 at the end of tile i and starts each tile without waiting
// for LDS.  The arithmetic and its order are those of scan_fwd_kernel, so
// both kernels give the same bits.
//
// Every tile is processed whole: the steps past the segment end are given
// delta = 0 (identity steps), so the saved state of a partial last chunk is
// the state at its last real step, and their outputs are never stored.
constexpr int kWsTile = 16;   // steps per tile
constexpr int kWsStage = 3;   // staging buffers (tiles i, i+1 and i+2)
constexpr int kWsRing = 4;    // producer register ring of raw rows, in tiles
constexpr int kCacheNT = 2;   // cache-policy bit NT (nontemporal) of a buffer access
static_assert(kWsTile == kChunk, "a tile is one saved chunk");

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));
typedef float f32x4_v __attribute__((ext_vector_type(4)));
static_assert(kWsProd * 4 == kWsTile, "one producer wave per 4-step column");
static_assert(2 * kWsCons * kWsTile == 64 * kWsProd, "one B/C value pair per producer lane");

// LDS column length of the role-split kernel, in float4s: 64 channel rows
// and 2 of padding, so consecutive columns start 1056 B apart (32 B past a
// multiple of the 128 B bank cycle).  The producers' 8-lane groups of a
// 128-bit access (rows r, r+1 x columns 0..3) then touch 8 distinct 16-byte
// bank groups, and the consumers' whole-column accesses are 64 consecutive
// float4s from one base register (the column is an immediate offset).
constexpr int kWsRow = kBlockCh + 2;

// One tile's raw loads of a producer lane, kept as loaded bits: converting
// at the load would make the compiler wait for it right there.
template <typename T, bool kDt = false>
struct WsRows {
  typename Raw4<T>::type u, d, z;
  uint32_t B, C;  // element bits
};
// With the fused step-size projection: the tile's dt^T operand in place of
// the delta row piece.
template <typename T>
struct WsRows<T, true> {
  typename Raw4<T>::type u, z;
  uint32_t B, C;
  u32x4_v pa[kDtK];
};


// kSum: the segment summaries instead of the scan (what scan_fwd_segsum_kernel
// computes, with the same bits): blockIdx.z is sub-segment j of seg_len /
// sub_k steps, the state starts from zero, the consumers run the recurrence
// without outputs or saves and leave the final state in seg_h, and the
// producers stage delta, delta*u and B/C only and sum the step sizes into
// seg_dt.  A producer lane keeps two sums, one over the even and one over the
// odd 16-step tiles of its 4-step column, and the four lanes of a channel row
// combine them as the summary kernel's eight lanes of 32-step tiles do
// (((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7)) over its columns c), so
// both kernels add the same numbers in the same order.
//
// kDt (1, or 2 to also store delta_raw to dtp.delta_out): delta_raw from the
// fused step-size projection (DtProj) instead of dl, and B / C from the token
// rows of dtp.params instead of Bp / Cp.
template <typename T, int kZ, bool kAligned, bool kSum, int kDt = 0>
__global__ __launch_bounds__(kWsThreads) void scan_fwd_ws_kernel(
    const ScanDims p, const T* __restrict__ u, const T* __restrict__ dl,
    const float* __restrict__ Ap, const T* __restrict__ Bp, const T* __restrict__ Cp,
    const float* __restrict__ Dp, const float* __restrict__ biasp,
    const float* __restrict__ h_init, const int64_t* __restrict__ length,
    const T* __restrict__ zp, T* __restrict__ out, T* __restrict__ yu,
    float* __restrict__ h_chunks, float* __restrict__ h_last, void* __restrict__ dummy,
    float* __restrict__ seg_h, float* __restrict__ seg_dt, const DtProj dtp) {
  static_assert(!kSum || kZ == 0, "the summaries read no gate");
  static_assert(!kDt || sizeof(T) == 2, "the fused projection reads bf16");
  static_assert(kDt != 2 || !kSum, "the summaries store no delta_raw");
  constexpr bool kDtOut = kDt == 2;
  constexpr bool kHasZ = kZ != 0;
  constexpr bool kSaveY = kZ == 2;
  constexpr int kT4 = kWsTile / 4;

  // [buffer][delta | delta * u][column][channel row]
  __shared__ float4 sSt[kWsStage][2][kT4][kWsRow];
  __shared__ float4 sBC[kWsStage][kWsCons][kWsTile];       // (B0, C0, B1, C1) per pair and step
  __shared__ float4 sY[2][kWsCons][kT4][kWsRow];           // per-wave partial sums of C*h
  // aligned rows: each producer wave's outputs of four tiles (its 16 rows x
  // 64 steps: one 128-byte line per row in bf16, two in fp32), as pieces of
  // 4 steps, [stream][row][tile][column], rows padded by 8 bytes
  using Piece = typename Raw4<T>::type;
  constexpr int kOutRowW = 16 * (int)sizeof(Piece) / 4 + 2;  // 32-bit words per padded row
  __shared__ uint32_t sOut[kAligned && !kSum ? kWsProd : 1][2][16 * kOutRowW];

  const int lane = threadIdx.x & 63;
  const int w = wave_id_uniform();
  const int b = blockIdx.y;
  const int d0 = blockIdx.x * kBlockCh;
  const int L = p.seqlen, Dm = p.dim, N = p.nstate;
  const int seg = blockIdx.z;
  // steps [Tbeg, Lend): segment seg, or with kSum summary part seg (whole
  // 32-step tiles, so pairs of 16-step tiles, up to the sequence end)
  int Tbeg, Lend;
  if constexpr (kSum) {
    sub_range(p, seg, Tbeg, Lend);
  } else {
    Tbeg = seg * p.seg_len;
    Lend = min(L, Tbeg + p.seg_len);
  }
  const int ntiles = max(0, (Lend - Tbeg + kWsTile - 1) / kWsTile);
  const size_t rb = (size_t)b * Dm;
  const size_t sb = (size_t)seg * p.batch + b;  // summary row (kSum)

  if (w < kWsCons) {
    // ------------------------------------------------ consumer: the recurrence
    const int ch = d0 + lane;
    const bool ch_ok = ch < Dm;
    float h[2], A2[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int n = 2 * w + s;
      const bool ok = ch_ok && n < N;
      A2[s] = ok ? Ap[(size_t)ch * N + n] * kLog2e : 0.0f;
      float hv = (!kSum && ok && h_init) ? h_init[(rb + ch) * N + n] : 0.0f;
      // carry in through the earlier summaries' affine maps, in order
      if (!kSum && ok)
        hv = fold_carry(hv, A2[s], seg_dt, seg_h, 0, 1, seg * p.sub_k, p.batch, b, Dm, N, n, ch);
      h[s] = hv;
    }
    const bool save = !kSum && h_chunks != nullptr;
    const size_t hsD = (size_t)p.hs * Dm;  // floats between the saved rows of two states
    const size_t cstride = (size_t)N * hsD;  // floats between the saves of two chunks
    // the saves go through a buffer range over the wave's two state rows of
    // the chunk: lanes past the last channel, and a second state past N,
    // get offsets outside it (the launch keeps 2 * hsD * 4 bytes < 2^31)
    float* const hc0 = save ? h_chunks + ((size_t)b * p.nchunks + Tbeg / kChunk) * cstride +
                                  (size_t)(2 * w) * hsD
                            : nullptr;
    const bool ok0 = ch_ok && 2 * w < N, ok1 = ch_ok && 2 * w + 1 < N;
    const uint32_t hoff0 = ok0 ? (uint32_t)ch * 4u : kOffDrop;
    const uint32_t hoff1 = ok1 ? (uint32_t)(hsD + ch) * 4u : kOffDrop;

    // block 0 of a tile: read at the end of the previous tile
    BC2 bcb[2];
    float4 dlb[2], dub[2];
    auto read_block = [&](int buf, int k, BC2& bc, float4& dl4, float4& du4) {
      lds_bc_block(sBC[buf][w], 4 * k, bc);
      const float4* __restrict__ st = &sSt[buf][0][0][lane];
      dl4 = st[k * kWsRow];
      du4 = st[(kT4 + k) * kWsRow];
    };
    // as many barriers as the producers: 1 + 4 * ceil(ntiles / 4)
    const int nbar = 1 + 4 * ((ntiles + 3) / 4);
    int buf = 0;
    for (int i = 0; i < nbar; ++i) {
      __syncthreads();
      if (i >= ntiles) continue;
      if (i == 0) read_block(0, 0, bcb[0], dlb[0], dub[0]);
      const int nbuf = buf == kWsStage - 1 ? 0 : buf + 1;
      float4* __restrict__ cY = &sY[i & 1][w][0][lane];
      // block k+1's LDS reads are issued before block k is computed; after
      // the last block, the next tile's first block (staged one iteration
      // ago, so complete since this tile's barrier)
#pragma unroll
      for (int k = 0; k < kT4; ++k) {
        const int c = k & 1;
        if (k + 1 < kT4) read_block(buf, k + 1, bcb[c ^ 1], dlb[c ^ 1], dub[c ^ 1]);
        else read_block(nbuf, 0, bcb[c ^ 1], dlb[c ^ 1], dub[c ^ 1]);
        if constexpr (kSum) {
          fwd_block_state(dlb[c], dub[c], bcb[c], A2, h);
        } else {
          float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
          fwd_block(dlb[c], dub[c], bcb[c], A2, h, y);
          cY[k * kWsRow] = make_float4(y[0], y[1], y[2], y[3]);
        }
      }
      // kT4 is even: the next tile's block 0 sits in buffer 0 again
      static_assert(kT4 % 2 == 0, "block 0 of every tile in register set 0");
      if (save) {
        // layout (batch, nchunks, nstate, dim): one contiguous 256 B run per
        // state; nontemporal, as the backward alone reads the saved states
        const auto hr = raw_rsrc(hc0 + (size_t)i * cstride, (uint32_t)(2 * hsD * sizeof(float)));
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(h[0]), hr, (int)hoff0, 0, kCacheNT);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(h[1]), hr, (int)hoff1, 0, kCacheNT);
      }
      buf = nbuf;
    }
    if constexpr (kSum) {
      if (ok0) seg_h[(sb * N + 2 * w) * Dm + ch] = h[0];
      if (ok1) seg_h[(sb * N + 2 * w + 1) * Dm + ch] = h[1];
    } else if (!save && h_last && Lend == L) {
      if (ok0) h_last[(rb + ch) * N + 2 * w] = h[0];
      if (ok1) h_last[(rb + ch) * N + 2 * w + 1] = h[1];
    }
    return;
  }

  // ------------------------------------------------ producer: staging and outputs
  // producer lane pt -> channel row pt / 4 and 4-step column q = pt % 4 of
  // every tile: the four lanes of a row read and write 16 consecutive steps
  const int pt = (w - kWsCons) * 64 + lane;
  // kDt: the layout of the projection's MFMA result, row lane % 16 of the
  // wave's 16 and column lane / 16, so each lane holds its own step sizes
  const int row = kDt ? (w - kWsCons) * (kBlockCh / kWsProd) + (lane & 15) : pt / kT4;
  const int q = kDt ? lane >> 4 : pt % kT4;
  const int pch = d0 + row;
  const bool pch_ok = pch < Dm;
  const float Dv = (pch_ok && Dp) ? Dp[pch] : 0.0f;
  const float Bias = (pch_ok && biasp) ? biasp[pch] : 0.0f;
  // rows of the clamped channel (valid addresses; lanes past the last channel
  // are masked to delta = 0 and never stored)
  const int chc = min(pch, Dm - 1);
  const T* __restrict__ u_row = u + (rb + chc) * L;
  const T* __restrict__ d_row = dl + (rb + chc) * L;
  // kDt: z's batch rows may lie dtp.zbstride elements apart (the gate half of
  // the in-projection output, read in place); zb offsets z so that the row
  // arithmetic below, which assumes dim * L, lands on them
  const T* __restrict__ zb = kDt ? zp + (size_t)b * dtp.zbstride - (size_t)rb * L : zp;
  const T* __restrict__ z_row = zb + (rb + chc) * L;
  int vlo, vhi;
  valid_window(length, p.pad_right, b, L, vlo, vhi);
  vhi = min(vhi, Lend);  // steps past the segment are identity steps here
  const bool softplus = p.softplus != 0;
  const int last_t0 = Tbeg + (ntiles - 1) * kWsTile;
  // B/C staging: producer lane pt -> (state 2G + half, step) of a tile.
  // With kDt B and C are token-major: a wave reads 4 steps x 16 states, so
  // one load touches 4 token rows (32 contiguous bytes each), not 16.
  const int bc_half = kDt ? lane & 1 : pt / (kWsCons * kWsTile);
  const int bc_G = kDt ? (lane >> 1) & 7 : (pt / kWsTile) % kWsCons;
  const int bc_step = kDt ? (w - kWsCons) * 4 + (lane >> 4) : pt % kWsTile;
  const int bc_n = 2 * bc_G + bc_half;
  const bool bc_ok = bc_n < N;
  const size_t bc_row = (size_t)b * p.bc_bstride + (size_t)min(bc_n, N - 1) * L;
  const T* __restrict__ B_row = Bp + bc_row;
  const T* __restrict__ C_row = Cp + bc_row;

  // raw rows of tile i (clamped to the last tile; the loads of tiles past it
  // are never used)
  // This wave's 16 channel rows (the launch guarantees 16 * L * sizeof(T) <
  // 2^31, so the byte offsets fit): the aligned path loads and stores through
  // buffer ranges over them, and loads B and C through ranges over the batch
  // row's state rows, at 32-bit offsets (no 64-bit address arithmetic per
  // tile).  The step is clamped into the row as on the pointer path; a row
  // past the last channel reads zero.
  const int wrow0 = d0 + (w - kWsCons) * (kBlockCh / kWsProd);
  const uint32_t wbytes =
      (uint32_t)(max(0, min(kBlockCh / kWsProd, Dm - wrow0)) * (size_t)L * sizeof(T));
  const uint32_t row_off = (uint32_t)((row % (kBlockCh / kWsProd)) * (size_t)L * sizeof(T));
  const auto u_ld = raw_rsrc(const_cast<T*>(u) + ((size_t)rb + wrow0) * L, wbytes);
  const auto d_ld = raw_rsrc(const_cast<T*>(dl) + ((size_t)rb + wrow0) * L, wbytes);
  const auto z_ld = raw_rsrc(kHasZ ? const_cast<T*>(zb) + ((size_t)rb + wrow0) * L : const_cast<T*>(u),
                             kHasZ ? wbytes : 0u);
  const uint32_t bc_bytes = (uint32_t)((size_t)N * L * sizeof(T));
  const auto B_ld = raw_rsrc(const_cast<T*>(Bp) + (size_t)b * p.bc_bstride, bc_bytes);
  const auto C_ld = raw_rsrc(const_cast<T*>(Cp) + (size_t)b * p.bc_bstride, bc_bytes);
  const uint32_t bc_row_off = (uint32_t)((size_t)min(bc_n, N - 1) * L * sizeof(T));

  // kDt: the batch row's token rows of params (the launch keeps L * P * 2 <
  // 2^31), this lane's byte offsets from a tile's first token row -- its
  // dt^T operand (token lane % 16; rank groups past the rank read group 0,
  // which meets zero weights) and its B / C values (token bc_step) -- and its
  // W_dt operand: channel d0 + 16 pw + lane % 16, ranks 32 s + 8 (lane / 16)
  // .. + 7, zero past the rank or the last channel.  Tokens past the end of
  // the sequence fall outside the buffer range and read zero: they are
  // identity steps, whose outputs are never stored.
  const uint32_t prow_bytes = kDt ? (uint32_t)dtp.P * 2u : 0u;
  const auto pr_ld =
      raw_rsrc(kDt ? static_cast<char*>(const_cast<void*>(dtp.params)) + (size_t)b * dtp.pstride * 2
                   : static_cast<char*>(dummy),
               (uint32_t)L * prow_bytes);
  uint32_t pa_off[kDtK] = {}, pbc_off = 0;
  bf16x8_v wdt[kDtK];
  if constexpr (kDt) {
    pbc_off = (uint32_t)bc_step * prow_bytes + (uint32_t)(dtp.rank + min(bc_n, N - 1)) * 2u;
    const int pw = w - kWsCons;
    const int wch = d0 + 16 * pw + (lane & 15);
    const __hip_bfloat16* wrow =
        static_cast<const __hip_bfloat16*>(dtp.w) + (size_t)min(wch, Dm - 1) * dtp.rank;
#pragma unroll
    for (int s = 0; s < kDtK; ++s) {
      const int g = 32 * s + 8 * (lane >> 4);
      const bool gok = g < dtp.rank;
      pa_off[s] = (uint32_t)(lane & 15) * prow_bytes + (uint32_t)(gok ? g : 0) * 2u;
      u32x4_v wv = {0u, 0u, 0u, 0u};
      if (gok && wch < Dm) wv = *reinterpret_cast<const u32x4_v*>(wrow + g);
      wdt[s] = __builtin_bit_cast(bf16x8_v, wv);
    }
  }

  auto issue = [&](WsRows<T, kDt != 0>& r, int i) {
    const int t0 = min(Tbeg + i * kWsTile, last_t0);
    if constexpr (kDt) {
      const uint32_t tb = (uint32_t)t0 * prow_bytes;  // wave-uniform
#pragma unroll
      for (int s = 0; s < kDtK; ++s)
        r.pa[s] = __builtin_amdgcn_raw_buffer_load_b128(pr_ld, (int)(tb + pa_off[s]), 0, 0);
      r.B = buffer_load_bits1<T>(pr_ld, tb + pbc_off);
      r.C = buffer_load_bits1<T>(pr_ld, tb + pbc_off + (uint32_t)N * 2u);
      if constexpr (kAligned) {
        const uint32_t off = row_off + (uint32_t)min(t0 + 4 * q, L - 4) * sizeof(T);
        r.u = buffer_load_raw4<T>(u_ld, off);
        if constexpr (kHasZ) r.z = buffer_load_raw4<T>(z_ld, off);
        else r.z = typename Raw4<T>::type{};
      } else {
        r.u = load_raw4_nb<T, kAligned>(u_row, t0 + 4 * q, L, pch_ok);
        if constexpr (kHasZ) r.z = load_raw4_nb<T, kAligned>(z_row, t0 + 4 * q, L, pch_ok);
        else r.z = typename Raw4<T>::type{};
      }
    } else if constexpr (kAligned) {
      const uint32_t off = row_off + (uint32_t)min(t0 + 4 * q, L - 4) * sizeof(T);
      r.u = buffer_load_raw4<T>(u_ld, off);
      r.d = buffer_load_raw4<T>(d_ld, off);
      if constexpr (kHasZ) r.z = buffer_load_raw4<T>(z_ld, off);
      else r.z = typename Raw4<T>::type{};
      const uint32_t boff = bc_row_off + (uint32_t)min(t0 + bc_step, L - 1) * sizeof(T);
      r.B = buffer_load_bits1<T>(B_ld, boff);
      r.C = buffer_load_bits1<T>(C_ld, boff);
    } else {
      r.u = load_raw4_nb<T, kAligned>(u_row, t0 + 4 * q, L, pch_ok);
      r.d = load_raw4_nb<T, kAligned>(d_row, t0 + 4 * q, L, pch_ok);
      if constexpr (kHasZ) r.z = load_raw4_nb<T, kAligned>(z_row, t0 + 4 * q, L, pch_ok);
      else r.z = typename Raw4<T>::type{};
      const int tb = min(t0 + bc_step, L - 1);
      r.B = elem_bits(B_row[tb]);
      r.C = elem_bits(C_row[tb]);
    }
  };

  // stage tile i into buffer sbuf: delta (softplus once per element, zero
  // outside the valid window), delta * u, B and C; D*u and silu(z) are kept
  // for its finish; with kSum, delta is also added to the sum of tile parity
  // par (i % 2)
  float dts[2] = {0.0f, 0.0f};  // kSum: step sizes of the even and odd tiles
  // kDtOut: the wave's 16 rows of delta_out (rows past the last channel lie
  // outside the range)
  const auto dto_rsrc =
      raw_rsrc(kDtOut ? static_cast<char*>(dtp.delta_out) + ((size_t)rb + wrow0) * L * sizeof(T)
                      : static_cast<char*>(dummy),
               kDtOut ? wbytes : 0u);
  // kDt: a tile's delta_raw (steps 4 (lane / 16) .. + 3 of channel lane % 16
  // of the wave's 16), issued an iteration before the tile is staged so that
  // the MFMA latency runs under that iteration's other work
  auto proj = [&](const WsRows<T, kDt != 0>& r) {
    f32x4_v acc = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (kDt) {
#pragma unroll
      for (int s = 0; s < kDtK; ++s)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_v, r.pa[s]), wdt[s],
                                                      acc, 0, 0, 0);
    }
    return acc;
  };
  auto stage = [&](const WsRows<T, kDt != 0>& r, const f32x4_v acc, int i, int sbuf, float (&sk)[4],
                   float (&gt)[4], int par) {
    const int t_tile = Tbeg + i * kWsTile;
    const int t = t_tile + 4 * q;
    float uv[4], dv[4], de[4], du[4];
    decode4(r.u, uv);
    if constexpr (kDt) {
      // this lane's row (channel lane % 16) and 4-step column (lane / 16),
      // rounded to bf16
      const uint32_t x01 = pack_bf16x2(acc[0], acc[1]);
      const uint32_t x23 = pack_bf16x2(acc[2], acc[3]);
      decode4(make_uint2(x01, x23), dv);
      if constexpr (kDtOut) {
        // delta_out (its own instantiation: a conditional path with memory
        // operations would make the compiler wait for the ring's loads at the
        // merge).  Aligned rows: L and the segment ends are multiples of 4,
        // so the 4 steps are one 8-byte piece inside the row or wholly past
        // its end.
        if constexpr (kAligned) {
          const uint32_t off = t < Lend ? row_off + (uint32_t)t * 2u : kOffDrop;
          const u32x2_v xv = {x01, x23};
          __builtin_amdgcn_raw_buffer_store_b64(xv, dto_rsrc, (int)off, 0, 0);
        } else {
          const uint32_t bits[4] = {x01 & 0xffffu, x01 >> 16, x23 & 0xffffu, x23 >> 16};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t off = t + j < Lend ? row_off + (uint32_t)(t + j) * 2u : kOffDrop;
            __builtin_amdgcn_raw_buffer_store_b16((unsigned short)bits[j], dto_rsrc, (int)off, 0, 0);
          }
        }
      }
    } else {
      decode4(r.d, dv);
    }
    if constexpr (kHasZ) {
      float zv[4];
      decode4(r.z, zv);
#pragma unroll
      for (int j = 0; j < 4; ++j) gt[j] = silu_f(zv[j]);
    }
    // Rows past the last channel are left unmasked: the consumer lanes that
    // read them store nothing.  Tiles wholly inside the valid window (all but
    // at most two per row) skip the window mask; the mask is a bitwise AND
    // rather than a select so that the compiler keeps the four elements in
    // one block instead of branching around the softplus of masked lanes.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      sk[j] = Dv * uv[j];
      const float x = dv[j] + Bias;
      const float sp = softplus_t20(x);
      de[j] = softplus ? sp : x;
    }
    if (!(t_tile >= vlo && t_tile + kWsTile <= vhi)) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t keep = (t + j >= vlo && t + j < vhi) ? 0xffffffffu : 0u;
        de[j] = __uint_as_float(__float_as_uint(de[j]) & keep);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) du[j] = de[j] * uv[j];
    if constexpr (kSum) {
#pragma unroll
      for (int j = 0; j < 4; ++j) dts[par] += de[j];
    }
    sSt[sbuf][0][q][row] = make_float4(de[0], de[1], de[2], de[3]);
    sSt[sbuf][1][q][row] = make_float4(du[0], du[1], du[2], du[3]);
    reinterpret_cast<float2*>(&sBC[sbuf][bc_G][bc_step])[bc_half] =
        bc_ok ? make_float2(bits_to_f32<T>(r.B), bits_to_f32<T>(r.C)) : make_float2(0.0f, 0.0f);
  };

  const auto out_rsrc = raw_rsrc(out + ((size_t)rb + wrow0) * L, wbytes);
  const auto yu_rsrc = raw_rsrc(kSaveY ? yu + ((size_t)rb + wrow0) * L : out, kSaveY ? wbytes : 0u);

  // finish tile i: the eight slices (read before the staging work of the
  // same iteration, added after it) in a fixed order, D*u, the gate, stores
  auto finish_read = [&](int i, float4 (&v)[kWsCons]) {
#pragma unroll
    for (int ww = 0; ww < kWsCons; ++ww) v[ww] = sY[i & 1][ww][q][row];
  };
  auto finish = [&](int i, const float4 (&v)[kWsCons], const float (&sk)[4],
                    const float (&gt)[4]) {
    const int t = Tbeg + i * kWsTile + 4 * q;
    float4 acc = v[0];
#pragma unroll
    for (int ww = 1; ww < kWsCons; ++ww) {
      acc.x += v[ww].x; acc.y += v[ww].y; acc.z += v[ww].z; acc.w += v[ww].w;
    }
    float y[4] = {sk[0] + acc.x, sk[1] + acc.y, sk[2] + acc.z, sk[3] + acc.w};
    if constexpr (kAligned) {
      // range-checked stores: rows past the last channel lie outside the
      // wave's buffer range, and steps past the segment get an offset past it
      const uint32_t off = t < Lend ? row_off + (uint32_t)t * sizeof(T) : kOffDrop;
      if constexpr (kSaveY) buffer_store4<T>(yu_rsrc, off, y);
      if constexpr (kHasZ) {
#pragma unroll
        for (int j = 0; j < 4; ++j) y[j] *= gt[j];
      }
      buffer_store4<T>(out_rsrc, off, y);
    } else {
      const bool st_ok = pch_ok && t < Lend;
      if constexpr (kSaveY) store4_nb<T, kAligned>(yu + (rb + pch) * L, t, L, st_ok, dummy, y);
      if constexpr (kHasZ) {
#pragma unroll
        for (int j = 0; j < 4; ++j) y[j] *= gt[j];
      }
      store4_nb<T, kAligned>(out + (rb + pch) * L, t, L, st_ok, dummy, y);
    }
  };

  // Aligned rows: the outputs of four consecutive tiles go to the wave's
  // LDS rows and are stored together, 16 bytes per lane and access, after
  // the fourth: each 64-step row piece is then written whole by back-to-back
  // stores (piece by piece, a line was completed over four tiles, and lines
  // evicted from L2 in between were written back more than once).
  const int prow = row % 16;  // this lane's row within the wave's 16
  const int pw = kAligned ? max(w - kWsCons, 0) : 0;
  uint32_t* const so_out = &sOut[pw][0][0];
  uint32_t* const so_yu = &sOut[pw][1][0];
  auto put_piece = [&](uint32_t* dst, const float (&y)[4]) {
    if constexpr (sizeof(T) == 2) {
      *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]));
    } else {
      // rows are 8-byte aligned only (padding), so two 8-byte writes
      reinterpret_cast<uint2*>(dst)[0] = make_uint2(__float_as_uint(y[0]), __float_as_uint(y[1]));
      reinterpret_cast<uint2*>(dst)[1] = make_uint2(__float_as_uint(y[2]), __float_as_uint(y[3]));
    }
  };
  auto finish_lds = [&](int i, const float4 (&v)[kWsCons], const float (&sk)[4],
                        const float (&gt)[4], int j) {
    float4 acc = v[0];
#pragma unroll
    for (int ww = 1; ww < kWsCons; ++ww) {
      acc.x += v[ww].x; acc.y += v[ww].y; acc.z += v[ww].z; acc.w += v[ww].w;
    }
    float y[4] = {sk[0] + acc.x, sk[1] + acc.y, sk[2] + acc.z, sk[3] + acc.w};
    const int slot = prow * kOutRowW + (4 * j + q) * (int)(sizeof(Piece) / 4);
    if constexpr (kSaveY) put_piece(so_yu + slot, y);
    if constexpr (kHasZ) {
#pragma unroll
      for (int k = 0; k < 4; ++k) y[k] *= gt[k];
    }
    put_piece(so_out + slot, y);
  };
  // tiles i - 3 .. i: the wave's 16 rows x 64 steps as 16-byte chunks, lane
  // l storing chunks l, l + 64, ...
  auto flush = [&](int i) {
    constexpr int kChunksRow = 64 * (int)sizeof(T) / 16;
    const int tl = Tbeg + (i - 3) * kWsTile;
#pragma unroll
    for (int m = 0; m < kChunksRow / 4; ++m) {
      const int c = lane + 64 * m;
      const int r = c / kChunksRow, pc = c % kChunksRow;
      const int t = tl + pc * (16 / (int)sizeof(T));
      const uint32_t off = t < Lend ? (uint32_t)((r * (size_t)L + t) * sizeof(T)) : kOffDrop;
      const int sw = r * kOutRowW + 4 * pc;
      const uint2* so = reinterpret_cast<const uint2*>(so_out + sw);
      const u32x4_v xo = {so[0].x, so[0].y, so[1].x, so[1].y};
      if constexpr (kSaveY) {
        const uint2* sy = reinterpret_cast<const uint2*>(so_yu + sw);
        const u32x4_v xy = {sy[0].x, sy[0].y, sy[1].x, sy[1].y};
        // the ungated output is read only by the backward: a nontemporal
        // store, which does not push the step's inputs out of the caches
        __builtin_amdgcn_raw_buffer_store_b128(xy, yu_rsrc, (int)off, 0, kCacheNT);
      }
      __builtin_amdgcn_raw_buffer_store_b128(xo, out_rsrc, (int)off, 0, 0);
    }
  };

  // Iteration i after barrier i: read tile i-1's slices (written during
  // iteration i-1), stage tile i+2 into buffer (i+2) % 3 (last read during
  // iteration i-1), finish tile i-1.  Raw rows travel in a ring of kWsRing
  // tiles: tile k's loads are issued when tile k - kWsRing is staged, kWsRing
  // iterations ahead of their use.  D*u and the gates ride in a ring of 4
  // tiles (staged at iteration k - 2, finished at k + 1).
  //
  // Iterations 1 .. 4m run in unrolled groups of four with no conditions
  // around memory operations: the compiler's wait for a ring slot's loads
  // then counts only the operations issued after them (a conditional path
  // into the loop header makes it wait for nearly all of them).  Work past
  // the last tile is harmless: its loads are clamped into the rows, its
  // staging buffers are never read and its stores fall outside the range.
  WsRows<T, kDt != 0> rows[kWsRing];
  float sk[4][4], gt[4][4];
  float4 v[kWsCons];
#pragma unroll
  for (int k = 0; k < kWsRing; ++k) issue(rows[k], k);
  stage(rows[0], proj(rows[0]), 0, 0, sk[0], gt[0], 0);
  issue(rows[0], kWsRing);
  stage(rows[1], proj(rows[1]), 1, 1, sk[1], gt[1], 1);
  issue(rows[1], kWsRing + 1);
  __syncthreads();  // iteration 0
  stage(rows[2], proj(rows[2]), 2, 2, sk[2], gt[2], 0);
  issue(rows[2], kWsRing + 2);
  f32x4_v dacc = proj(rows[3]);  // kDt: tile 3, staged at iteration 1
  int sbuf = 0;  // staging buffer of tile i + 2
  for (int i0 = 1; i0 <= ntiles; i0 += 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = i0 + j;  // (i + 2) % 4 == (j + 3) % 4, (i - 1) % 4 == j
      __syncthreads();
      if constexpr (!kSum) finish_read(i - 1, v);
      // i0 % 4 == 1, so tile i + 2 has the parity of j + 3
      stage(rows[(j + 3) % kWsRing], dacc, i + 2, sbuf, sk[(j + 3) & 3], gt[(j + 3) & 3],
            (j + 3) & 1);
      issue(rows[(j + 3) % kWsRing], i + 2 + kWsRing);
      if constexpr (!kSum) {
        if constexpr (kAligned) {
          finish_lds(i - 1, v, sk[j], gt[j], j);
          if (j == 3) flush(i - 1);
        } else {
          finish(i - 1, v, sk[j], gt[j]);
        }
      }
      // tile i + 3 sits in ring slot (i + 3) % 4 == j
      dacc = proj(rows[j]);
      sbuf = sbuf == kWsStage - 1 ? 0 : sbuf + 1;
    }
  }
  if constexpr (kSum) {
    // the four lanes of a channel row: 4 consecutive lanes (q = lane % 4), or
    // with kDt lanes 16 apart (q = lane / 16); either way columns 0+1 and 2+3
    // first, then their sums
#pragma unroll
    for (int m = 1; m < kT4; m <<= 1) {
      const int x = kDt ? 16 * m : m;
      dts[0] += __shfl_xor(dts[0], x, 64);
      dts[1] += __shfl_xor(dts[1], x, 64);
    }
    if (q == 0 && pch_ok) seg_dt[sb * Dm + pch] = dts[0] + dts[1];
  }
}

// ---------------------------------------------------------------- segment summaries

// For sub-segment j = blockIdx.z (seg_len / sub_k steps; the sub-segments
// cover segments 0 .. nseg - 2) of batch row b and 64 channels: the state the
// sub-segment's steps produce from zero, h_seg = sum_t (prod_{t' > t} a_t')
// delta_t u_t B_t, and its summed step size sum_t delta_t (padded steps count
// zero), the two numbers that let a later segment start from the right state.
// Finer sub-segments than segments keep the device full when the segments
// alone would leave CUs idle (few batch rows x channel blocks).  The same tiling as the forward (64 channels x 32
// steps per tile, lane = channel, wave = state pair) without outputs: phase A
// stages delta and delta*u in LDS (double-buffered by tile parity, so one
// barrier per tile suffices), phase B runs the recurrence with B read as
// wave-uniform values of the prepped layout.
template <typename T, int kSG, bool kAligned>
__global__ __launch_bounds__(kThreads) void scan_fwd_segsum_kernel(
    const ScanDims p, const T* __restrict__ u, const T* __restrict__ dl,
    const float* __restrict__ Ap, const float* __restrict__ bc, const float* __restrict__ biasp,
    const int64_t* __restrict__ length, float* __restrict__ seg_h, float* __restrict__ seg_dt) {
  using R4 = typename Raw4<T>::type;
  constexpr int kT4 = kTileF / 4;
  static_assert(kBlockCh * kT4 == kThreads, "one 4-step row piece per thread");
  __shared__ float4 sDelta[2][kT4][kBlockCh];
  __shared__ float4 sDu[2][kT4][kBlockCh];
  __shared__ float4 sB[2][kWaves][kTileF / 2];  // (B0, B1) of steps 2i, 2i+1 per pair

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = wave_id_uniform();
  const int b = blockIdx.y;
  const int d0 = blockIdx.x * kBlockCh;
  const int seg = blockIdx.z;  // summary part
  const int L = p.seqlen, Dm = p.dim, N = p.nstate;
  int Tbeg, Lend;
  sub_range(p, seg, Tbeg, Lend);
  const int npair = bc_pairs(N);
  const int Lp = bc_row_len(L);
  const size_t rb = (size_t)b * Dm;
  int vlo, vhi;
  valid_window(length, p.pad_right, b, L, vlo, vhi);

  const int ch = d0 + lane;
  const bool ch_ok = ch < Dm;
  float h[kSG][2], A2[kSG][2];
#pragma unroll
  for (int g = 0; g < kSG; ++g)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int n = (g * kWaves + w) * 2 + s;
      A2[g][s] = (ch_ok && n < N) ? Ap[(size_t)ch * N + n] * kLog2e : 0.0f;
      h[g][s] = 0.0f;
    }

  const int a_row = tid / kT4;
  const int a_q = tid % kT4;
  const int a_col = a_q * 4;
  const int a_sw = a_row ^ col_swz(a_q);
  const int a_ch = d0 + a_row;
  const bool a_ok = a_ch < Dm;
  const float Bias = (a_ok && biasp) ? biasp[a_ch] : 0.0f;
  const int a_chc = min(a_ch, Dm - 1);
  const T* __restrict__ u_row = u + (rb + a_chc) * L;
  const T* __restrict__ d_row = dl + (rb + a_chc) * L;
  const bool softplus = p.softplus != 0;
  const int last_t0 = (Lend - 1) / kTileF * kTileF;
  const float4* __restrict__ bc4 = reinterpret_cast<const float4*>(bc);
  float dtsum = 0.0f;

  // B staging (kSG == 1): thread tid < 256 owns (pair tid / 32, step tid % 32)
  const int bc_G = (tid / kTileF) % kWaves;
  const int bc_t = tid % kTileF;
  auto load_b = [&](int T0) {
    const int t = min(T0 + bc_t, Lp - 1);
    return bc4[((size_t)b * npair + bc_G) * Lp + t];
  };
  R4 qu = load_raw4_nb<T, kAligned>(u_row, Tbeg + a_col, L, a_ok);
  R4 qd = load_raw4_nb<T, kAligned>(d_row, Tbeg + a_col, L, a_ok);
  float4 qb = kSG == 1 ? load_b(Tbeg) : make_float4(0.f, 0.f, 0.f, 0.f);
  int buf = 0;
  for (int T0 = Tbeg; T0 < Lend; T0 += kTileF) {
    {
      float uv[4], dv[4], de[4], du[4];
      decode4(qu, uv);
      decode4(qd, dv);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float x = dv[j] + Bias;
        const float dt = softplus ? softplus_t20(x) : x;
        const int tt = T0 + a_col + j;
        const bool valid = a_ok && tt >= vlo && tt < vhi && tt < Lend;
        de[j] = valid ? dt : 0.0f;
        du[j] = de[j] * uv[j];
        dtsum += de[j];
      }
      sDelta[buf][a_q][a_sw] = make_float4(de[0], de[1], de[2], de[3]);
      sDu[buf][a_q][a_sw] = make_float4(du[0], du[1], du[2], du[3]);
      if (kSG == 1 && tid < kWaves * kTileF) {
        // (B0, B1) of this step into the pair's row: two steps per float4
        float* row = reinterpret_cast<float*>(&sB[buf][bc_G][0]);
        row[2 * bc_t] = qb.x;
        row[2 * bc_t + 1] = qb.z;
      }
    }
    // next tile's rows (the last tile re-reads itself)
    const int Tn = min(T0 + kTileF, last_t0);
    qu = load_raw4_nb<T, kAligned>(u_row, Tn + a_col, L, a_ok);
    qd = load_raw4_nb<T, kAligned>(d_row, Tn + a_col, L, a_ok);
    if constexpr (kSG == 1) qb = load_b(Tn);
    __syncthreads();
    const int nT4 = min(kT4, (Lend - T0 + 3) / 4);
    if (kSG == 1 && nT4 == kT4) {
      // full tile: 8 blocks unrolled, each block's LDS reads one block ahead
      const float4* __restrict__ bro = sB[buf][w];
      float4 dlb[2], dub[2], bb[2][2];
      dlb[0] = sDelta[buf][0][lane ^ col_swz(0)];
      dub[0] = sDu[buf][0][lane ^ col_swz(0)];
      bb[0][0] = bro[0];
      bb[0][1] = bro[1];
#pragma unroll
      for (int k = 0; k < kT4; ++k) {
        const int c = k & 1;
        if (k + 1 < kT4) {
          dlb[c ^ 1] = sDelta[buf][k + 1][lane ^ col_swz(k + 1)];
          dub[c ^ 1] = sDu[buf][k + 1][lane ^ col_swz(k + 1)];
          bb[c ^ 1][0] = bro[2 * (k + 1)];
          bb[c ^ 1][1] = bro[2 * (k + 1) + 1];
        }
        const float dlv[4] = {dlb[c].x, dlb[c].y, dlb[c].z, dlb[c].w};
        const float duv[4] = {dub[c].x, dub[c].y, dub[c].z, dub[c].w};
        const float b0[4] = {bb[c][0].x, bb[c][0].z, bb[c][1].x, bb[c][1].z};
        const float b1[4] = {bb[c][0].y, bb[c][0].w, bb[c][1].y, bb[c][1].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          h[0][0] = fmaf(fast_exp2(dlv[j] * A2[0][0]), h[0][0], duv[j] * b0[j]);
          h[0][1] = fmaf(fast_exp2(dlv[j] * A2[0][1]), h[0][1], duv[j] * b1[j]);
        }
      }
      buf ^= 1;
      continue;
    }
    for (int t4 = 0; t4 < nT4; ++t4) {
      const float4 dl4 = sDelta[buf][t4][lane ^ col_swz(t4)];
      const float4 du4 = sDu[buf][t4][lane ^ col_swz(t4)];
      const float dlv[4] = {dl4.x, dl4.y, dl4.z, dl4.w};
      const float duv[4] = {du4.x, du4.y, du4.z, du4.w};
      const int tb = T0 + 4 * t4;
#pragma unroll
      for (int g = 0; g < kSG; ++g) {
        const int G = g * kWaves + w;
        if (G < npair) {
          const float4* __restrict__ q = bc4 + ((size_t)b * npair + G) * Lp + tb;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float4 v = q[j];  // (B0, C0, B1, C1), wave-uniform
            h[g][0] = fmaf(fast_exp2(dlv[j] * A2[g][0]), h[g][0], duv[j] * v.x);
            h[g][1] = fmaf(fast_exp2(dlv[j] * A2[g][1]), h[g][1], duv[j] * v.z);
          }
        }
      }
    }
    buf ^= 1;
  }

  const size_t sb = (size_t)seg * p.batch + b;
  if (ch_ok) {
#pragma unroll
    for (int g = 0; g < kSG; ++g)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int n = (g * kWaves + w) * 2 + s;
        if (n < N) seg_h[(sb * N + n) * Dm + ch] = h[g][s];
      }
  }
  // the 8 threads of a channel row are 8 consecutive lanes
#pragma unroll
  for (int m = 1; m < kT4; m <<= 1) dtsum += __shfl_xor(dtsum, m, 64);
  if (a_q == 0 && a_ok) seg_dt[sb * Dm + a_ch] = dtsum;
}

// ---------------------------------------------------------------- chunk decays

// The first half of the reference's (prod a, h) chunk carry
// (csrc/selective_scan/forward_kernel.cu:225-228), whose chunks are
// kRefChunk = 128 steps (kernel_config.h:4-10): the product of the decays
// a_t = exp(delta_t A) from step 0 to the end of each 128-step chunk c, which
// is exp(A * S_c) with S_c the sum of the step sizes over those steps (padded
// steps count zero, as their decay is 1).  The pair layout pairs
// (batch, nchunks, 2 * nstate, dim) fp32 has nchunks = kRefSlots * (number of
// 128-step chunks) slots of 16 steps: the scan writes the states into the odd
// rows of slots 0 .. ceil(seqlen / 16) - 1, and chunk c's carry is slot
// kRefSlots * c + kRefSlots - 1, the last 16-step slot of the chunk.  The
// decays go into that slot's even rows, by two kernels that run before the
// scan; when seqlen is not a multiple of 128 the last chunk's carry slot lies
// past the last state the scan writes, and chunk_tail_kernel copies the final
// state there after the scan.
constexpr int kRefChunk = 128;
constexpr int kRefSlots = kRefChunk / kChunk;

__device__ __forceinline__ size_t ref_slot(int c) { return (size_t)c * kRefSlots + kRefSlots - 1; }

// Step-size sum of each 128-step chunk, per (b, d, chunk c), parked in the
// odd row of state 0 of the chunk's carry slot (the scan, or the tail copy,
// overwrites it); consecutive threads take consecutive chunks of a row.
template <typename T>
__global__ __launch_bounds__(256) void chunk_dt_sum_kernel(const ScanDims p,
                                                           const T* __restrict__ dl,
                                                           const float* __restrict__ biasp,
                                                           const int64_t* __restrict__ length,
                                                           float* __restrict__ pairs) {
  const int L = p.seqlen, Dm = p.dim, N2 = 2 * p.nstate;
  const int slots = p.nchunks, K = slots / kRefSlots;
  const size_t total = (size_t)p.batch * Dm * K;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const int c = (int)(i % K);
    const size_t bd = i / K;
    const int d = (int)(bd % Dm), b = (int)(bd / Dm);
    int vlo, vhi;
    valid_window(length, p.pad_right, b, L, vlo, vhi);
    const float bias = biasp ? biasp[d] : 0.0f;
    const T* row = dl + bd * L;
    const int t1 = min(L, (c + 1) * kRefChunk);
    float acc = 0.0f;
    for (int t = c * kRefChunk; t < t1; ++t) {
      const float x = Elem<T>::load1(row + t) + bias;
      const float dt = p.softplus ? softplus_t20(x) : x;
      acc += (t >= vlo && t < vhi) ? dt : 0.0f;
    }
    pairs[(((size_t)b * slots + ref_slot(c)) * N2 + 1) * Dm + d] = acc;
  }
}

// prod a per (b, d, state n) at every 128-step chunk end: a running sum of
// the chunk step sums, and exp2(A log2(e) S) into the even rows of the
// chunk's carry slot.  One thread per (b, d, group of 4 states);
// consecutive threads take consecutive channels, so the writes are
// contiguous.
__global__ __launch_bounds__(256) void chunk_decay_kernel(const ScanDims p,
                                                          const float* __restrict__ Ap,
                                                          float* __restrict__ pairs) {
  const int Dm = p.dim, slots = p.nchunks, K = slots / kRefSlots, N = p.nstate, N2 = 2 * N;
  const int ng = (N + 3) / 4;
  const size_t total = (size_t)p.batch * ng * Dm;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const int d = (int)(i % Dm);
    const size_t r = i / Dm;
    const int q = (int)(r % ng), b = (int)(r / ng);
    float A2[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = 4 * q + j;
      A2[j] = n < N ? Ap[(size_t)d * N + n] * kLog2e : 0.0f;
    }
    float S = 0.0f;
    for (int c = 0; c < K; ++c) {
      float* slot = pairs + ((size_t)b * slots + ref_slot(c)) * N2 * Dm + d;
      S += slot[Dm];  // the chunk's step sum (odd row of state 0)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = 4 * q + j;
        if (n < N) slot[(size_t)2 * n * Dm] = fast_exp2(A2[j] * S);
      }
    }
  }
}

// After the scan, when the last 128-step chunk is partial: its carry slot
// receives the final state (odd rows of the last slot the scan wrote).  One
// thread per (b, n, d).
__global__ __launch_bounds__(256) void chunk_tail_kernel(const ScanDims p, float* __restrict__ pairs) {
  const int Dm = p.dim, N = p.nstate, N2 = 2 * N, slots = p.nchunks;
  const int last = (p.seqlen + kChunk - 1) / kChunk - 1;
  const size_t total = (size_t)p.batch * N * Dm;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const int d = (int)(i % Dm);
    const size_t r = i / Dm;
    const int n = (int)(r % N), b = (int)(r / N);
    const size_t row = (size_t)(2 * n + 1) * Dm + d;
    pairs[((size_t)b * slots + slots - 1) * N2 * Dm + row] =
        pairs[((size_t)b * slots + last) * N2 * Dm + row];
  }
}

hipError_t launch_chunk_decay(const ScanParams& p, int dtype, float* pairs, hipStream_t st) {
  const size_t n1 = (size_t)p.batch * p.dim * (p.nchunks / kRefSlots);
  {
    ProfScope prof("chunk_dt_sum", st);
    const int blocks = (int)std::min<size_t>((n1 + 255) / 256, 65535);
    if (dtype == 1)
      hipLaunchKernelGGL(chunk_dt_sum_kernel<__hip_bfloat16>, dim3(blocks), dim3(256), 0, st,
                         dims_of(p), (const __hip_bfloat16*)p.delta, p.bias, p.length, pairs);
    else
      hipLaunchKernelGGL(chunk_dt_sum_kernel<float>, dim3(blocks), dim3(256), 0, st, dims_of(p),
                         (const float*)p.delta, p.bias, p.length, pairs);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  ProfScope prof("chunk_decay", st);
  const size_t n2 = (size_t)p.batch * ((p.nstate + 3) / 4) * p.dim;
  const int blocks = (int)std::min<size_t>((n2 + 255) / 256, 65535);
  hipLaunchKernelGGL(chunk_decay_kernel, dim3(blocks), dim3(256), 0, st, dims_of(p), p.A, pairs);
  return hipGetLastError();
}

hipError_t launch_chunk_tail(const ScanParams& p, float* pairs, hipStream_t st) {
  if ((p.seqlen + kChunk - 1) / kChunk == p.nchunks) return hipSuccess;  // 128 | seqlen
  ProfScope prof("chunk_tail", st);
  const size_t n = (size_t)p.batch * p.nstate * p.dim;
  const int blocks = (int)std::min<size_t>((n + 255) / 256, 65535);
  hipLaunchKernelGGL(chunk_tail_kernel, dim3(blocks), dim3(256), 0, st, dims_of(p), pairs);
  return hipGetLastError();
}

// ---------------------------------------------------------------- launch

size_t bc_prep_floats(int batch, int nstate, int seqlen) {
  return (size_t)batch * bc_pairs(nstate) * bc_row_len(seqlen) * 4;
}

// Segments of the forward sequence split: enough for about one workgroup per
// compute unit of the 256-CU gfx950 (every workgroup holds a CU's worth of
// LDS), each a whole number of super-tiles; 1 when the batch and channel
// blocks already fill the device.
void fwd_segments(int batch, int nblk, int seqlen, int& nseg, int& seg_len) {
  constexpr int kSup = kSubF * kTileF;
  constexpr int kTargetWG = 256, kMaxSeg = 16;
  const int rows = batch * nblk;
  int s = rows >= kTargetWG ? 1 : kTargetWG / rows;
  s = std::max(1, std::min({s, kMaxSeg, (seqlen + kSup - 1) / kSup}));
  seg_len = ((seqlen + s - 1) / s + kSup - 1) / kSup * kSup;
  nseg = (seqlen + seg_len - 1) / seg_len;
}

// Summary parts per segment (the forward's cover segments 0 .. nseg - 2, the
// backward's 1 .. nseg - 1; sub_span steps each, sub_range).  The summary
// kernels are VALU-bound and a CU holds two of their workgroups, so with k
// parts the busiest CU runs about ceil(workgroups / CUs) of them one after
// the other, each sub_span steps plus a pipeline start-up of about kStartup
// steps (the loads of the first tiles): k = 1 .. 8 is picked for the least
// such cost, the smaller k on a tie.
int fwd_summary_split(int batch, int nblk, int nseg, int seg_len) {
  constexpr long kCUs = 256;
  constexpr int kStartup = 64, kMaxK = 8;
  if (nseg <= 1) return 1;
  const long wg = (long)(nseg - 1) * batch * nblk;
  int best = 1;
  long best_cost = (wg + kCUs - 1) / kCUs * (seg_len + kStartup);
  for (int k = 2; k <= kMaxK; ++k) {
    const long cost = (wg * k + kCUs - 1) / kCUs * (sub_span(seg_len, k) + kStartup);
    if (cost < best_cost) {
      best = k;
      best_cost = cost;
    }
  }
  return best;
}

size_t fwd_seg_floats(int batch, int dim, int nstate, int seqlen) {
  int nseg, seg_len;
  const int nblk = (dim + kBlockCh - 1) / kBlockCh;
  fwd_segments(batch, nblk, seqlen, nseg, seg_len);
  const int k = fwd_summary_split(batch, nblk, nseg, seg_len);
  return (size_t)(nseg - 1) * k * batch * dim * (nstate + 1);
}

hipError_t launch_bc_prep(const ScanParams& p, int dtype, float* bc, hipStream_t st) {
  const int npair = bc_pairs(p.nstate);
  const int Lp = bc_row_len(p.seqlen);
  const size_t total = (size_t)p.batch * npair * Lp;
  const int blocks = (int)std::min<size_t>((total + 255) / 256, 65535);
  ProfScope prof("bc_prep", st);
  if (dtype == 1)
    hipLaunchKernelGGL(bc_prep_kernel<__hip_bfloat16>, dim3(blocks), dim3(256), 0, st, p.batch,
                       p.nstate, p.seqlen, npair, Lp, (const __hip_bfloat16*)p.B,
                       (const __hip_bfloat16*)p.C, p.bc_bstride, bc);
  else
    hipLaunchKernelGGL(bc_prep_kernel<float>, dim3(blocks), dim3(256), 0, st, p.batch, p.nstate,
                       p.seqlen, npair, Lp, (const float*)p.B, (const float*)p.C, p.bc_bstride, bc);
  return hipGetLastError();
}

// The role-split forward serves N <= 16 when its buffer ranges fit 2^31
// bytes (a wave's 16 rows of output, 16 * L * elem, and a wave's two saved
// state rows, 2 * hs * dim * 4); the general kernel serves the rest.
static bool ws_forward(const ScanParams& p, size_t elem) {
  return p.nstate <= 16 && (size_t)(kBlockCh / kWsProd) * p.seqlen * elem < (1u << 31) &&
         (size_t)2 * p.hs * p.dim * sizeof(float) < (1u << 31);
}

template <typename T, int kSG, int kZ, bool kAligned>
static hipError_t launch_fwd4(const ScanParams& p, const float* bc, hipStream_t st) {
  const bool ws = ws_forward(p, sizeof(T));
  if (p.nseg > 1) {
    ProfScope prof("scan_fwd_segsum", st);
    if (ws)
      hipLaunchKernelGGL((scan_fwd_ws_kernel<T, 0, kAligned, true>),
                         dim3(p.nblk, p.batch, (p.nseg - 1) * p.sub_k), dim3(kWsThreads), 0, st,
                         dims_of(p), (const T*)p.u, (const T*)p.delta, p.A, (const T*)p.B,
                         (const T*)p.C, p.D, p.bias, p.h_init, p.length, (const T*)nullptr,
                         (T*)p.out, (T*)nullptr, (float*)nullptr, (float*)nullptr, p.dummy,
                         p.seg_h, p.seg_dt, DtProj{});
    else
      hipLaunchKernelGGL((scan_fwd_segsum_kernel<T, kSG, kAligned>),
                         dim3(p.nblk, p.batch, (p.nseg - 1) * p.sub_k), dim3(kThreads), 0, st,
                         dims_of(p),
                         (const T*)p.u, (const T*)p.delta, p.A, bc, p.bias, p.length, p.seg_h,
                         p.seg_dt);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  ProfScope prof("scan_fwd", st);
  if (ws) {
    hipLaunchKernelGGL((scan_fwd_ws_kernel<T, kZ, kAligned, false>), dim3(p.nblk, p.batch, p.nseg),
                       dim3(kWsThreads), 0, st, dims_of(p), (const T*)p.u, (const T*)p.delta, p.A,
                       (const T*)p.B, (const T*)p.C, p.D, p.bias, p.h_init, p.length,
                       (const T*)p.z, (T*)p.out, (T*)p.out_ungated, p.h_chunks, p.h_last, p.dummy,
                       p.seg_h, p.seg_dt, DtProj{});
    return hipGetLastError();
  }
  hipLaunchKernelGGL((scan_fwd_kernel<T, kSG, kZ, kAligned>),
                     dim3(p.nblk, p.batch, p.nseg), dim3(kThreads), 0, st, dims_of(p),
                     (const T*)p.u, (const T*)p.delta, p.A, bc, (const T*)p.B, (const T*)p.C, p.D,
                     p.bias, p.h_init, p.length, (const T*)p.z, (T*)p.out, (T*)p.out_ungated,
                     p.h_chunks, p.h_last, p.dummy, p.seg_h, p.seg_dt);
  return hipGetLastError();
}

template <typename T, int kSG>
static hipError_t launch_fwd3(const ScanParams& p, const float* bc, bool aligned, hipStream_t st) {
  if (p.z && p.out_ungated)
    return aligned ? launch_fwd4<T, kSG, 2, true>(p, bc, st)
                   : launch_fwd4<T, kSG, 2, false>(p, bc, st);
  if (p.z)
    return aligned ? launch_fwd4<T, kSG, 1, true>(p, bc, st)
                   : launch_fwd4<T, kSG, 1, false>(p, bc, st);
  return aligned ? launch_fwd4<T, kSG, 0, true>(p, bc, st)
                 : launch_fwd4<T, kSG, 0, false>(p, bc, st);
}

template <typename T>
static hipError_t launch_fwd2(const ScanParams& p, const float* bc, bool aligned, hipStream_t st) {
  if (p.nstate <= 16) return launch_fwd3<T, 1>(p, bc, aligned, st);
  if (p.nstate <= 32) return launch_fwd3<T, 2>(p, bc, aligned, st);
  if (p.nstate <= 64) return launch_fwd3<T, 4>(p, bc, aligned, st);
  return launch_fwd3<T, 16>(p, bc, aligned, st);
}

// The prepped B/C layout serves state counts past 16 and the general
// kernel's segment summaries; the role-split kernels read B and C directly.
static bool fwd_needs_bc_prep(const ScanParams& p, size_t elem) {
  return p.nstate > 16 || (p.nseg > 1 && !ws_forward(p, elem));
}

// bc must hold bc_prep_floats() floats; it is filled here before the scan
// when a kernel reads the prepped layout.
hipError_t launch_scan_fwd(const ScanParams& p, int dtype, bool aligned, float* bc,
                           hipStream_t st) {
  if (fwd_needs_bc_prep(p, dtype == 1 ? 2 : 4)) {
    hipError_t e = launch_bc_prep(p, dtype, bc, st);
    if (e != hipSuccess) return e;
  }
  if (dtype == 1) return launch_fwd2<__hip_bfloat16>(p, bc, aligned, st);
  return launch_fwd2<float>(p, bc, aligned, st);
}

// The forward with the fused step-size projection (DtProj): bf16, the
// role-split kernel only.  p.delta, p.B and p.C are not read; the kernels'
// delta, B and C arguments get valid addresses they never load from.
bool scan_fwd_dt_supported(const ScanParams& p) { return p.nstate <= 16 && ws_forward(p, 2); }

template <int kZ, bool kAligned, bool kSum, int kDt>
static void launch_ws_dt(const ScanParams& p, const DtProj& dt, hipStream_t st) {
  using T = __hip_bfloat16;
  const int gz = kSum ? (p.nseg - 1) * p.sub_k : p.nseg;
  const T* prm = static_cast<const T*>(dt.params);
  hipLaunchKernelGGL((scan_fwd_ws_kernel<T, kZ, kAligned, kSum, kDt>), dim3(p.nblk, p.batch, gz),
                     dim3(kWsThreads), 0, st, dims_of(p), (const T*)p.u, (const T*)p.u, p.A, prm,
                     prm, p.D, p.bias, p.h_init, p.length, (const T*)p.z, (T*)p.out,
                     (T*)nullptr, (float*)nullptr, p.h_last, p.dummy, p.seg_h, p.seg_dt, dt);
}

hipError_t launch_scan_fwd_dt(const ScanParams& p, const DtProj& dt, bool aligned, hipStream_t st) {
  if (p.nseg > 1) {
    ProfScope prof("scan_fwd_segsum", st);
    if (aligned) launch_ws_dt<0, true, true, 1>(p, dt, st);
    else launch_ws_dt<0, false, true, 1>(p, dt, st);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  ProfScope prof("scan_fwd", st);
  // with delta_out, the instantiation that stores it
  const int k = (p.z ? 2 : 0) + (aligned ? 1 : 0) + (dt.delta_out ? 4 : 0);
  switch (k) {
    case 0: launch_ws_dt<0, false, false, 1>(p, dt, st); break;
    case 1: launch_ws_dt<0, true, false, 1>(p, dt, st); break;
    case 2: launch_ws_dt<1, false, false, 1>(p, dt, st); break;
    case 3: launch_ws_dt<1, true, false, 1>(p, dt, st); break;
    case 4: launch_ws_dt<0, false, false, 2>(p, dt, st); break;
    case 5: launch_ws_dt<0, true, false, 2>(p, dt, st); break;
    case 6: launch_ws_dt<1, false, false, 2>(p, dt, st); break;
    default: launch_ws_dt<1, true, false, 2>(p, dt, st); break;
  }
  return hipGetLastError();
}

}  // namespace ssm
