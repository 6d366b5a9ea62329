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
// dz = dy * y * silu'(z) with y the forward's ungated output (saved by the
// forward, so the backward does not recompute sum_n C h) and dy unmasked: the
// gate is the caller's elementwise product outside the scan
// (modules/mamba.py:181-182), which autograd differentiates at every
// position, padded ones included.
//
// Work decomposition mirrors the forward (workgroup = batch row b x 64
// channels, 8 waves, lane = channel, wave w = state pairs G = g*8 + w).  Tiles
// of 16 steps (one saved-state chunk) are walked from the end.  For each tile
// a wave reloads the state the forward saved at the tile start, recomputes the
// 16 states and decay factors of its two states into registers, then runs the
// reverse recurrence.  The tile's B and C are read straight from B and C (one
// element per thread, coalesced along the steps, a tile ahead), parked in LDS
// in block-register order, and each wave takes its 4-step blocks from there
// as block registers read through DPP row broadcasts.  Per-position
// sums over states (sum G B, sum A G a h) leave each wave in its own
// LDS slice and are added in a fixed order; the per-position sums over
// channels (dB, dC) are reduced across the 64 lanes with a permlane/DPP
// reduce-scatter (two 4-step blocks at a time in the role-split kernel) and
// written as one partial per (channel block, b, n, t), in rows padded to whole
// tiles, which a second small kernel adds up.  dA, dD and dbias are written as
// per-batch-row partials reduced by the same kernel, so the result is
// deterministic (no atomics).
#include <type_traits>

#include "ss_io.cuh"
#include "ss_params.h"
#include "ss_prof.h"

namespace ssm {

namespace {

// Row length of the dB/dC partials: seqlen padded to whole 16-step tiles, so
// a tile's stores need no step check (the padding is never read).
__host__ __device__ __forceinline__ int bc_part_len(int L) { return (L + kTileB - 1) / kTileB * kTileB; }

// softplus and its derivative with the reference's threshold 20, as
// softplus_and_grad_t20, without the select of the derivative above the
// threshold: there e = exp(-x) < 2^-24, so 1 + e rounds to 1 and its
// reciprocal is 1 exactly, the value the threshold gives.
__device__ __forceinline__ void softplus_and_grad_u(float x, float& sp, float& sg) {
  const float e = fast_exp2(-fabsf(x) * kLog2e);
  const float r = fast_rcp(1.0f + e);
  sp = fmaxf(x, 0.0f) + log1p_pos(e);
  sg = x >= 0.0f ? r : e * r;
}

// Reduce-scatter folds on lane bits 3 and 2 without selects: two DPP adds
// with complementary bank masks write one register, the lanes whose bit is
// clear adding the pair's first value with their partner's, the others the
// second (the sums rs_fold forms, in the same operand order up to
// commutation, so the same bits).  Banks are lane bits 3..2 of a row.  A DPP
// read needs two wait states after a VALU write of its source, which the
// compiler does not see inside the asm: fold_ror8's s_nop provides them where
// its inputs may be the products computed just before; fold_ror8_nn, for
// inputs computed a block's reverse earlier, and fold_half_mirror, which reads
// fold_ror8 results of the level before, go without (an s_nop per fold cost
// the backward 1.7%).  tests/test_dpp_hazards.py checks the compiled kernels
// for any DPP source written by VALU within two wait states.
__device__ __forceinline__ float fold_ror8(float p, float q) {  // bit 3: partner l ^ 8
  float r;
  asm("s_nop 1\n\t"
      "v_add_f32_dpp %0, %1, %1 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %0, %2, %2 row_ror:8 row_mask:0xf bank_mask:0xc"
      : "=&v"(r)
      : "v"(p), "v"(q));
  return r;
}
__device__ __forceinline__ float fold_ror8_nn(float p, float q) {  // fold_ror8 without the s_nop
  float r;
  asm("v_add_f32_dpp %0, %1, %1 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %0, %2, %2 row_ror:8 row_mask:0xf bank_mask:0xc"
      : "=&v"(r)
      : "v"(p), "v"(q));
  return r;
}
// Four fold_ror8 at once behind one s_nop: the two wait states cover every
// input of the block.
__device__ __forceinline__ void fold_ror8_x4(float (&v)[32], int i0) {
  float r0, r1, r2, r3;
  asm("s_nop 1\n\t"
      "v_add_f32_dpp %0, %4, %4 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %0, %5, %5 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
      "v_add_f32_dpp %1, %6, %6 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %1, %7, %7 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
      "v_add_f32_dpp %2, %8, %8 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %2, %9, %9 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
      "v_add_f32_dpp %3, %10, %10 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %3, %11, %11 row_ror:8 row_mask:0xf bank_mask:0xc"
      : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3)
      : "v"(v[i0]), "v"(v[i0 + 16]), "v"(v[i0 + 1]), "v"(v[i0 + 17]), "v"(v[i0 + 2]),
        "v"(v[i0 + 18]), "v"(v[i0 + 3]), "v"(v[i0 + 19]));
  v[i0] = r0; v[i0 + 1] = r1; v[i0 + 2] = r2; v[i0 + 3] = r3;
}
__device__ __forceinline__ float fold_half_mirror(float p, float q) {  // bit 2: partner 7 - l in 8
  float r;
  asm("v_add_f32_dpp %0, %1, %1 row_half_mirror row_mask:0xf bank_mask:0x5\n\t"
      "v_add_f32_dpp %0, %2, %2 row_half_mirror row_mask:0xf bank_mask:0xa"
      : "=&v"(r)
      : "v"(p), "v"(q));
  return r;
}

// Sum over the 64 lanes of 32 values per lane.  The cross-row moves
// (v_permlane16/32_swap) cost about 2.4 issue slots each against 1 for the
// in-row DPP forms (measured), so the in-row folds go first, on 32 and 16
// values, and the swaps after them, on 8 and 4:
//   lane bit 3 (row_ror:8, masked) -> value bit 4,
//   lane bit 2 (row_half_mirror, masked; the partner 7 - l also differs in
//     bits 1..0, which the last two levels sum over) -> value bit 3,
//   lane bit 4 (permlane16 swaps) -> value bit 2,
//   lane bit 5 (permlane32 swaps) -> value bit 1,
//   lane bit 1 (quad_perm xor 2, with selects) -> value bit 0,
// then an add over lane bit 0.  Afterwards v[0] of lane l holds the total of
// value index (b3 b2 b4 b5 b1) of l's bits (lanes l and l ^ 1 hold the same):
// 64 VALU with 6 swaps, against 70 with 24 for the permlane levels first.
__device__ __forceinline__ int reduce32_index(int lane) {
  return ((lane >> 3) & 1) << 4 | ((lane >> 2) & 1) << 3 | ((lane >> 4) & 1) << 2 |
         ((lane >> 5) & 1) << 1 | ((lane >> 1) & 1);
}
// kOld: the values were computed well before the call (no fresh VALU
// results), so the first level's folds go without their s_nop; otherwise
// they run four to an asm block behind one s_nop.
template <bool kOld = false>
__device__ __forceinline__ void wave_reduce32(float (&v)[32], int lane) {
  if constexpr (kOld) {
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = fold_ror8_nn(v[i], v[i + 16]);
  } else {
#pragma unroll
    for (int i = 0; i < 16; i += 4) fold_ror8_x4(v, i);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = fold_half_mirror(v[i], v[i + 8]);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]), __float_as_uint(v[i + 4]),
                                              false, false);
    v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[i + 2]),
                                              false, false);
    v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  v[0] = rs_fold<kDppQuadXor2>(v[0], v[1], (lane & 2) != 0);
  v[0] += dpp_mov<kDppQuadXor1>(v[0]);
}

struct StepVals {  // per-position LDS values of one 4-step block
  float4 dl, du, dout;
};

// The reverse recurrence needs the decays a_t of the tile: keep the 32 values
// from the recompute in registers, or recompute them (one mul and one exp per
// state and step) and save the registers.
#ifndef SSM_BWD_RECOMPUTE_DECAY
#define SSM_BWD_RECOMPUTE_DECAY 0
#endif
constexpr bool kRecomputeDecay = SSM_BWD_RECOMPUTE_DECAY != 0;

// B/C of a 4-step block for the wave's state pair, as a block register
// (lane l holds value l & 15 of the prepped block [j][s][B, C]).
__device__ __forceinline__ int kB(int j, int s) { return j * 4 + s * 2; }
__device__ __forceinline__ int kC(int j, int s) { return j * 4 + s * 2 + 1; }

// Recompute one 4-step block: decays a and states H for the wave's 2 states.
__device__ __forceinline__ void bwd_recompute_block(int jq, const StepVals& sv, float blk,
                                                    const float (&A2)[2], const float (&Hc)[2],
                                                    float (&a)[2][kChunk], float (&H)[2][kChunk],
                                                    float (&y)[4]) {
  const float dlv[4] = {sv.dl.x, sv.dl.y, sv.dl.z, sv.dl.w};
  const float duv[4] = {sv.du.x, sv.du.y, sv.du.z, sv.du.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = 4 * jq + j;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const float at = fast_exp2(dlv[j] * A2[s]);
      if constexpr (!kRecomputeDecay) a[s][i] = at;
      const float hp = i ? H[s][i - 1] : Hc[s];
      H[s][i] = fmaf(at, hp, bc_mul(kB(j, s), blk, duv[j]));
      y[j] = s == 0 ? bc_mul(kC(j, s), blk, H[s][i]) : bc_fmac(kC(j, s), y[j], blk, H[s][i]);
    }
  }
}

// Reverse recurrence over one 4-step block (steps 4jq+3 .. 4jq).  vals gets
// the block's per-channel terms of dB (index s*4 + j) and dC (8 + s*4 + j),
// to be summed over the 64 channels of the wave.
__device__ __forceinline__ void bwd_reverse_block(int jq, const StepVals& sv, float blk,
                                                  const float (&Av)[2], const float (&A2)[2],
                                                  const float (&Hc)[2],
                                                  const float (&a)[2][kChunk],
                                                  const float (&H)[2][kChunk], float (&gam)[2],
                                                  float (&dA)[2], float (&vals)[16],
                                                  float (&gB)[4], float (&gD)[4]) {
  const float dlv[4] = {sv.dl.x, sv.dl.y, sv.dl.z, sv.dl.w};
  const float duv[4] = {sv.du.x, sv.du.y, sv.du.z, sv.du.w};
  const float dov[4] = {sv.dout.x, sv.dout.y, sv.dout.z, sv.dout.w};
#pragma unroll
  for (int j = 3; j >= 0; --j) {
    const int i = 4 * jq + j;
    float sB = 0.0f, sD = 0.0f;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const float Gt = bc_fmac(kC(j, s), gam[s], blk, dov[j]);  // gamma + dout C
      sB = s == 0 ? bc_mul(kB(j, s), blk, Gt) : bc_fmac(kB(j, s), sB, blk, Gt);
      const float hp = i ? H[s][i - 1] : Hc[s];
      const float at = kRecomputeDecay ? fast_exp2(dlv[j] * A2[s]) : a[s][i];
      const float ng = at * Gt;  // gamma_{t-1}
      const float q = ng * hp;        // G_t a_t h_{t-1}
      sD = fmaf(Av[s], q, sD);
      dA[s] = fmaf(dlv[j], q, dA[s]);
      vals[s * 4 + j] = Gt * duv[j];            // dB term
      vals[8 + s * 4 + j] = dov[j] * H[s][i];   // dC term
      gam[s] = ng;
    }
    gB[j] = sB;
    gD[j] = sD;
  }
}

}  // namespace

// LDS column swizzle of the 4-column (16-step) tiles: (row, column q) is
// stored at row index row ^ bcol_swz(q).  The tile-phase threads access 4
// columns of 16 rows per wave, and without the swizzle the columns (1 KiB
// apart) share banks; with it every 8- or 16-lane group of a 128-bit LDS
// access touches distinct banks.  Phase B reads whole columns (permutations of
// 64 consecutive float4s).
__device__ __forceinline__ constexpr int bcol_swz(int q) { return 4 * q + 2 * (q >> 1); }

// two elements of an aligned row (the unaligned path keeps element stores)
template <typename T, bool kAligned>
__device__ __forceinline__ void store2_nb(T* __restrict__ row, int t, int L, bool ok,
                                          void* __restrict__ dummy, const float (&v)[4]) {
  if constexpr (kAligned) {
    T* dst = (ok && t < L) ? row + t : static_cast<T*>(dummy);
    if constexpr (sizeof(T) == 4) {
      *reinterpret_cast<float2*>(dst) = make_float2(v[0], v[1]);
    } else {
      *reinterpret_cast<uint32_t*>(dst) = pack_bf16x2(v[0], v[1]);
    }
  } else {
    if (ok) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
        if (t + j < L) Elem<T>::store1(row + t + j, v[j]);
    }
  }
}

//
// kPart (state counts past 64): the workgroup covers the 64 states of state
// chunk sc = blockIdx.z / nseg (blockIdx.z % nseg is the segment) and writes
// its per-position sums over those states, sum_n G B and sum_n A G a h, as
// fp32 partials (ws_gb, ws_gd: (nsc, batch, dim, seqlen)); du, ddelta, dD
// and dbias then come from scan_bwd_combine_kernel, which adds the chunks'
// partials in a fixed order.  dz (state-independent) is written by chunk 0.
template <typename T, int kSG, bool kHasZ, bool kAligned, bool kPart>
__global__ __launch_bounds__(kThreads) void scan_bwd_kernel(
    const ScanDims p, const T* __restrict__ u, const T* __restrict__ dl,
    const float* __restrict__ Ap, const T* __restrict__ Bp, const T* __restrict__ Cp,
    const float* __restrict__ Dp, const float* __restrict__ biasp,
    const float* __restrict__ h_init, const int64_t* __restrict__ length,
    const T* __restrict__ zp, const T* __restrict__ yup, const float* __restrict__ h_chunks,
    const T* __restrict__ dyp,
    const float* __restrict__ dh_last, T* __restrict__ dup, T* __restrict__ ddp,
    T* __restrict__ dzp, float* __restrict__ dh_init, float* __restrict__ ws_bc,
    float* __restrict__ ws_A, float* __restrict__ ws_D, float* __restrict__ ws_bias,
    void* __restrict__ dummy, const float* __restrict__ seg_g, const float* __restrict__ seg_dt,
    float* __restrict__ ws_gb, float* __restrict__ ws_gd) {
  using R4 = typename Raw4<T>::type;
  constexpr int kT4 = kTileB / 4;         // 4-step columns per tile (4)
  constexpr int kItems = kBlockCh * kT4;  // (row, column) items per tile (256)
  static_assert(2 * kItems == kThreads, "two thread groups of one item each");
  static_assert(kTileB == kChunk, "one saved state per backward tile");
  constexpr int kMaxPairs = kSG * kWaves;  // state pairs covered by the dispatch bucket
  static_assert(kMaxPairs * kTileB <= kThreads, "one B/C float4 per thread per tile");

  __shared__ float4 sDelta[kT4][kBlockCh];  // delta (0 at padded steps)
  __shared__ float4 sDu[kT4][kBlockCh];     // delta * u
  // sDout, sU and sSg are written in phase A by one thread group and read in
  // phase C by the other, with no barrier between a tile's phase C and the
  // next tile's phase A: they alternate between two buffers by tile parity
  __shared__ float4 sSg[2][kT4][kBlockCh];  // softplus'(x) (0 at padded steps)
  __shared__ float4 sDout[2][kT4][kBlockCh];  // masked dout (after the z gate)
  __shared__ float4 sU[2][kT4][kBlockCh];
  // one slice per wave of the per-position sums over that wave's states,
  // added in a fixed order in phase C (deterministic result)
  __shared__ float4 sGB[kWaves][kT4][kBlockCh];  // sum_n G B
  __shared__ float4 sDD[kWaves][kT4][kBlockCh];  // sum_n A G a h_{t-1}

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = wave_id_uniform();
  const int b = blockIdx.y;
  const int blk = blockIdx.x;
  const int d0 = blk * kBlockCh;
  const int L = p.seqlen, Dm = p.dim, N = p.nstate;
  // sequence split: this workgroup's tiles [tile_beg, tile_end) of segment
  // seg; state chunk sc (kPart) covers states n0 .. n0 + 2 * kWaves * kSG - 1
  const int seg = kPart ? (int)blockIdx.z % p.nseg : (int)blockIdx.z;
  const int sc = kPart ? (int)blockIdx.z / p.nseg : 0;
  const int n0 = sc * (2 * kWaves * kSG);
  const int ntiles = (L + kTileB - 1) / kTileB;
  const int tile_beg = seg * (p.seg_len / kTileB);
  const int tile_end = min(ntiles, tile_beg + p.seg_len / kTileB);
  const size_t srow = (size_t)seg * p.batch + b;  // (segment, batch row) of the partials
  const int ngroups = (N + 1) / 2;
  const size_t rb = (size_t)b * Dm;
  const int Lp = bc_part_len(L);  // partial rows padded to whole tiles
  const size_t nBC = (size_t)p.batch * N * Lp;
  const T* __restrict__ Braw = Bp + (size_t)b * p.bc_bstride;
  const T* __restrict__ Craw = Cp + (size_t)b * p.bc_bstride;
  float* const dummyf = static_cast<float*>(dummy);

  int vlo, vhi;
  valid_window(length, p.pad_right, b, L, vlo, vhi);

  const int ch = d0 + lane;
  const bool ch_ok = ch < Dm;

  // persistent per-state values: reverse carry gamma and dA accumulator
  float gam[kSG][2], dA[kSG][2], Av[kSG][2], A2[kSG][2];
#pragma unroll
  for (int g = 0; g < kSG; ++g)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int n = n0 + (g * kWaves + w) * 2 + s;
      const bool ok = ch_ok && n < N;
      dA[g][s] = 0.0f;
      Av[g][s] = ok ? Ap[(size_t)ch * N + n] : 0.0f;
      A2[g][s] = Av[g][s] * kLog2e;
      // carry in from the later segments, last first:
      // gamma <- gamma_seg + exp(A sum dt) gamma (their summaries, zero carry-in)
      // (summary row k = segment k + 1, k = nseg - 2 .. seg)
      float q = (ok && dh_last) ? dh_last[(rb + ch) * N + n] : 0.0f;
      if (ok)
        q = fold_carry(q, A2[g][s], seg_dt, seg_g, p.nseg - 2, -1, p.nseg - 1 - seg, p.batch, b, Dm,
                       N, n, ch);
      gam[g][s] = q;
    }

  // ---- tile-phase mapping.  Group 0 (waves 0-3) owns the u / delta side
  // (softplus and staging, then du and dD); group 1 (waves 4-7) the dout / z
  // side (the gate, staging dout, dz), then ddelta and dbias.  Item =
  // (channel row, 4 consecutive steps) in both groups.
  const bool grp1 = w >= kWaves / 2;
  const int item = tid % kItems;
  const int a_row = item / kT4;
  const int a_q = item % kT4;
  const int a_col = a_q * 4;
  const int a_sw = a_row ^ bcol_swz(a_q);
  const int a_ch = d0 + a_row;
  const bool a_ok = a_ch < Dm;
  const int a_chc = min(a_ch, Dm - 1);
  const float Dv = (a_ok && Dp) ? Dp[a_ch] : 0.0f;
  const float Bias = (a_ok && biasp) ? biasp[a_ch] : 0.0f;
  const bool load2 = !grp1 || kHasZ;
  const T* __restrict__ row1 = (grp1 ? dyp : u) + (rb + a_chc) * L;
  const T* __restrict__ row2 = load2 ? (grp1 ? zp : dl) + (rb + a_chc) * L : row1;
  // group 1: the ungated forward output (group 0 re-reads its u row, so both
  // groups issue the same memory operations)
  const T* __restrict__ row3 = (kHasZ && grp1) ? yup + (rb + a_chc) * L : row1;
  const bool softplus = p.softplus != 0;
  const uint32_t okm = a_ok ? 0xffffffffu : 0u;
  float accD = 0.0f, accB = 0.0f;

  // Prefetch of a tile's inputs.  Every load is unconditional from a
  // clamped, valid address (masks are applied where the values are used):
  // a branch around a load, or a select on a value right after it, makes the
  // compiler wait for outstanding memory operations there.
  R4 n1, n2, n3;        // raw row pieces (group 0: u, delta; group 1: dout, z, y)
  float hcn[kSG][2];    // states saved by the forward before the tile
  // B and C of the next tile: thread i reads element i (and i + 512, ...)
  // of the tile's (B|C, state, step) set, coalesced along the steps;
  // phase A parks it in LDS in block-register order and phase B takes the
  // wave's 4-step blocks from there
  constexpr int kBCStates = 2 * kWaves * kSG;  // states covered by the dispatch bucket
  static_assert(2 * kBCStates * kTileB == kSG * kThreads, "kSG B/C elements per thread");
  __shared__ float sBlk[kWaves * kSG][kT4][16];  // [pair][block][(step, state, B|C)]
  T bcn[kSG];  // as loaded: converting at the load would make the compiler wait there
  const int chc = min(ch, Dm - 1);
  auto issue = [&](int tile) {
    const int t = tile * kTileB + a_col;
    n1 = load_raw4_nb<T, kAligned>(row1, t, L, a_ok);
    n2 = load_raw4_nb<T, kAligned>(row2, t, L, a_ok);
    if constexpr (kHasZ) n3 = load_raw4_nb<T, kAligned>(row3, t, L, a_ok);
#pragma unroll
    for (int g = 0; g < kSG; ++g) {
      // element e = (B|C, state, step) of the tile, clamped into the rows
      // (states past N are zeroed in phase A, steps past L meet delta = 0)
      const int e = g * kThreads + tid;
      const int n = min(n0 + (e / kTileB) % kBCStates, N - 1);
      const int t = min(tile * kTileB + e % kTileB, L - 1);
      bcn[g] = ((e / (kTileB * kBCStates)) ? Craw : Braw)[(size_t)n * L + t];
    }
#pragma unroll
    for (int g = 0; g < kSG; ++g)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int nc = min(n0 + (g * kWaves + w) * 2 + s, N - 1);
        const float* src = tile > 0
            ? h_chunks + (((size_t)b * p.nchunks + (tile - 1)) * N + nc) * p.hs * (size_t)Dm + chc
            : (h_init ? h_init + (rb + chc) * N + nc : h_chunks);
        hcn[g][s] = *src;
      }
  };

  float hc[kSG][2];
  float dzo[4];  // group 1: dz of the tile, stored at the start of phase C
  // ---- phase A: stage a tile's per-position quantities in LDS and take its
  // saved states and B/C blocks
  auto phase_a = [&](const int tile) {
    const int t0 = tile * kTileB;
    const int par = tile & 1;
    float v1[4], v2[4];
    decode4(n1, v1);
    decode4(n2, v2);
    // Masks (channel past the last one, step outside the valid window) are
    // bitwise ANDs rather than selects, and the softplus switch selects its
    // result: either way the compiler keeps the four elements in one block
    // instead of branching around the transcendental work of masked lanes.
    uint32_t keep[4] = {okm, okm, okm, okm};
    if (!(t0 >= vlo && t0 + kTileB <= vhi)) {  // tiles wholly inside the window skip this
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tt = t0 + a_col + j;
        keep[j] = (a_ok && tt >= vlo && tt < vhi) ? 0xffffffffu : 0u;
      }
    }
    if (!grp1) {  // u = v1, delta_raw = v2
      float de[4], du[4], sg[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float x = v2[j] + Bias;
        float sp, g;
        softplus_and_grad_t20(x, sp, g);
        de[j] = __uint_as_float(__float_as_uint(softplus ? sp : x) & keep[j]);
        sg[j] = __uint_as_float(__float_as_uint(softplus ? g : 1.0f) & keep[j]);
        du[j] = de[j] * v1[j];
      }
      sDelta[a_q][a_sw] = make_float4(de[0], de[1], de[2], de[3]);
      sDu[a_q][a_sw] = make_float4(du[0], du[1], du[2], du[3]);
      sU[par][a_q][a_sw] = make_float4(v1[0], v1[1], v1[2], v1[3]);
      sSg[par][a_q][a_sw] = make_float4(sg[0], sg[1], sg[2], sg[3]);
    } else {  // dy = v1, z = v2, y = v3
      float dov[4], v3[4];
      if constexpr (kHasZ) decode4(n3, v3);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float dym = __uint_as_float(__float_as_uint(v1[j]) & keep[j]);
        if constexpr (kHasZ) {
          const float sz = sigmoidf_fast(v2[j]);
          dov[j] = dym * (v2[j] * sz);
          dzo[j] = v1[j] * v3[j] * (sz * fmaf(v2[j], 1.0f - sz, 1.0f));  // every position
        } else {
          dov[j] = dym;
          dzo[j] = 0.0f;
        }
      }
      sDout[par][a_q][a_sw] = make_float4(dov[0], dov[1], dov[2], dov[3]);
    }
#pragma unroll
    for (int g = 0; g < kSG; ++g) {
      const int e = g * kThreads + tid;
      const int j = e % kTileB, n = (e / kTileB) % kBCStates, kind = e / (kTileB * kBCStates);
      sBlk[n >> 1][j >> 2][(j & 3) * 4 + (n & 1) * 2 + kind] = n0 + n < N ? to_f32(bcn[g]) : 0.0f;
    }
#pragma unroll
    for (int g = 0; g < kSG; ++g)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int n = n0 + (g * kWaves + w) * 2 + s;
        hc[g][s] = (ch_ok && n < N && (tile > 0 || h_init)) ? hcn[g][s] : 0.0f;
      }
  };

  // ---- phase B: recompute the tile's states, then the reverse recurrence
  auto phase_b = [&](const int tile) {
    const int t0 = tile * kTileB;
    const int par = tile & 1;
#pragma unroll
    for (int g = 0; g < kSG; ++g) {
      const int G = g * kWaves + w;
      if (g > 0 && n0 / 2 + G >= ngroups) {  // wave-uniform (pairs n0/2 + 0..7 always run: zero B/C)
        continue;
      }
      float a[2][kChunk], H[2][kChunk];
      StepVals X, Y;
      float bcg[kT4];  // block registers of the wave's pair G: lane l holds value l & 15
#pragma unroll
      for (int jq = 0; jq < kT4; ++jq) bcg[jq] = sBlk[G][jq][lane & 15];
      // slice update: the first group writes, later groups add
      auto put4 = [&](float4 (&slice)[kT4][kBlockCh], int q, const float (&v)[4]) {
        float4& dst = slice[q][lane ^ bcol_swz(q)];
        if (g == 0) {
          dst = make_float4(v[0], v[1], v[2], v[3]);
        } else {
          const float4 o = dst;
          dst = make_float4(o.x + v[0], o.y + v[1], o.z + v[2], o.w + v[3]);
        }
      };
      auto fwd = [&](int jq, const StepVals& sv) {
        float y[4];  // unused here (the forward saved the output)
        bwd_recompute_block(jq, sv, bcg[jq], A2[g], hc[g], a, H, y);
      };
      // the value of lane l after the reduction: index l >> 2 of the block's
      // 16 (kind = dB/dC, state, step); quads hold the same value
      const int vi = lane >> 2;
      const int rkind = vi >> 3, rs = (vi >> 2) & 1, rj = vi & 3;
      const int rn = n0 + G * 2 + rs;
      float* const wsb = ws_bc + ((size_t)rkind * p.nblk + blk) * nBC + ((size_t)b * N + rn) * Lp;
      auto rev = [&](int jq, const StepVals& sv) {
        float gB[4], gD[4], vals[16];
        bwd_reverse_block(jq, sv, bcg[jq], Av[g], A2[g], hc[g], a, H, gam[g], dA[g], vals, gB,
                          gD);
        put4(sGB[w], jq, gB);
        put4(sDD[w], jq, gD);
        // sum over the 64 channels of this block
        wave_reduce16(vals, lane);
        const int t = t0 + 4 * jq + rj;
        *((rn < N && t < L) ? wsb + t : dummyf) = vals[0];
      };
      auto ld = [&](int jq, StepVals& sv, bool with_dout) {
        const int li = lane ^ bcol_swz(jq);
        sv.dl = sDelta[jq][li];
        sv.du = sDu[jq][li];
        if (with_dout) sv.dout = sDout[par][jq][li];
      };
      // fixed schedule F0 F1 F2 F3 R3 R2 R1 R0 (recompute, then reverse); LDS
      // reads return in order, so the compiler overlaps them with the math
      ld(0, X, false); fwd(0, X);
      ld(1, Y, false); fwd(1, Y);
      ld(2, X, false); fwd(2, X);
      ld(3, Y, true);  fwd(3, Y);
      // the reverse re-reads the block registers: hide their values from
      // the recompute's, so each DPP broadcast folds into its own multiply
      // (shared, it is materialised with an extra v_mov_dpp and a register)
#pragma unroll
      for (int jq = 0; jq < kT4; ++jq) asm volatile("" : "+v"(bcg[jq]));
      rev(3, Y);
      ld(2, X, true); rev(2, X);
      ld(1, Y, true); rev(1, Y);
      ld(0, X, true); rev(0, X);
    }
  };

  // ---- phase C: per-position gradients.  Both groups add the slices of
  // sum_n G B; group 0 then writes du (and accumulates dD), group 1 writes
  // dz, adds the slices of sum_n A G a h as well and writes ddelta (and
  // accumulates dbias).  Two stores each (group 0 writes du as two halves),
  // so every path has the same memory-operation count; the split evens out
  // the work of the two groups between the barriers (group 0 also runs the
  // softplus in phase A, group 1 the gate).
  // Waves w and w + 4 share a SIMD, so an uneven split leaves each SIMD with
  // one wave to issue from.
  auto phase_c = [&](const int tile) {
    const int t0 = tile * kTileB;
    const int par = tile & 1;
    const int t = t0 + a_col;
    // group 1 writes the dz it computed in phase A first
    if (grp1) store4_nb<T, kAligned>(dzp + (rb + a_ch) * L, t, L, kHasZ && a_ok && sc == 0, dummy,
                                     dzo);
    if constexpr (kPart) {
      // the chunk's per-position sums over its states, fp32
      float4 acc = grp1 ? sDD[0][a_q][a_sw] : sGB[0][a_q][a_sw];
#pragma unroll
      for (int ww = 1; ww < kWaves; ++ww) {
        const float4 q1 = grp1 ? sDD[ww][a_q][a_sw] : sGB[ww][a_q][a_sw];
        acc.x += q1.x; acc.y += q1.y; acc.z += q1.z; acc.w += q1.w;
      }
      const float av[4] = {acc.x, acc.y, acc.z, acc.w};
      float* dst = (grp1 ? ws_gd : ws_gb) + (((size_t)sc * p.batch + b) * Dm + a_chc) * L;
      store4_nb<float, kAligned>(dst, t, L, a_ok, dummy, av);
      return;
    }
    float4 gb = sGB[0][a_q][a_sw];
#pragma unroll
    for (int ww = 1; ww < kWaves; ++ww) {
      const float4 q1 = sGB[ww][a_q][a_sw];
      gb.x += q1.x; gb.y += q1.y; gb.z += q1.z; gb.w += q1.w;
    }
    const float gbv[4] = {gb.x, gb.y, gb.z, gb.w};
    float uu[4];
    f4_to(sU[par][a_q][a_sw], uu);
    if (!grp1) {
      float de[4], dov[4];
      f4_to(sDelta[a_q][a_sw], de);
      f4_to(sDout[par][a_q][a_sw], dov);
      float duo[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        duo[j] = fmaf(Dv, dov[j], de[j] * gbv[j]);
        accD = fmaf(dov[j], uu[j], accD);  // dov is 0 at padded steps
      }
      // as two stores, so both groups issue two in phase C
      const float du0[4] = {duo[0], duo[1], 0.0f, 0.0f};
      const float du1[4] = {duo[2], duo[3], 0.0f, 0.0f};
      store2_nb<T, kAligned>(dup + (rb + a_ch) * L, t, L, a_ok, dummy, du0);
      store2_nb<T, kAligned>(dup + (rb + a_ch) * L, t + 2, L, a_ok, dummy, du1);
    } else {
      float4 gd = sDD[0][a_q][a_sw];
#pragma unroll
      for (int ww = 1; ww < kWaves; ++ww) {
        const float4 q2 = sDD[ww][a_q][a_sw];
        gd.x += q2.x; gd.y += q2.y; gd.z += q2.z; gd.w += q2.w;
      }
      const float gdv[4] = {gd.x, gd.y, gd.z, gd.w};
      float sg[4];
      f4_to(sSg[par][a_q][a_sw], sg);
      float ddo[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ddo[j] = fmaf(uu[j], gbv[j], gdv[j]) * sg[j];  // sg is 0 at padded steps
        accB += ddo[j];
      }
      store4_nb<T, kAligned>(ddp + (rb + a_ch) * L, t, L, a_ok, dummy, ddo);
    }
  };

  // Rotated loop: a tile's phase A (which waits for its prefetched inputs)
  // runs at the end of the previous iteration, in the same iteration as the
  // loads and the stores issued after them, so the waits count exactly.
  issue(tile_end - 1);
  phase_a(tile_end - 1);
  for (int tile = tile_end - 1; tile >= tile_beg; --tile) {
    __syncthreads();
    issue(max(tile - 1, tile_beg));  // at the first tile the tile itself is re-read, unused
    phase_b(tile);
    __syncthreads();
    phase_c(tile);
    if (tile > tile_beg) phase_a(tile - 1);
    // the next phase B overwrites the slices only after the barrier at the
    // top of the next iteration
  }

  // ---- per-row partials
#pragma unroll
  for (int g = 0; g < kSG; ++g)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int n = n0 + (g * kWaves + w) * 2 + s;
      if (ch_ok && n < N) {
        ws_A[(srow * Dm + ch) * N + n] = dA[g][s];
        if (dh_init && seg == 0) dh_init[(rb + ch) * N + n] = gam[g][s];
      }
    }
  // the 4 items of a channel row are 4 consecutive lanes of a group: dD
  // from group 0, dbias from group 1 (kPart: scan_bwd_combine_kernel)
  if constexpr (!kPart) {
    const float sv = group_sum<kT4>(grp1 ? accB : accD);
    if (a_ok && a_q == 0) (grp1 ? ws_bias : ws_D)[srow * Dm + a_ch] = sv;
  }
}

// ---------------------------------------------------------------- backward, N <= 16

// Role-split backward for up to 16 states, the counterpart of the forward's
// role split.  A workgroup of 12 waves covers one batch row b x 64 channels
// and walks its segment's 16-step tiles from the end:
//   consumer waves 0..7   lane = channel, wave w = states 2w and 2w+1: take
//                         the state the forward saved before the tile,
//                         recompute the tile's 16 states and decays, run the
//                         reverse recurrence, leave the per-position sums
//                         over the wave's states (sum_n G B, sum_n A G a h) in
//                         the wave's LDS slices, and write the dB / dC terms
//                         summed over the 64 channels;
//   producer waves 8..11  lane -> (channel row, 4-step column): stage the next
//                         tile (delta and softplus'(x) once per element,
//                         delta * u, the masked and gated dout, B and C) and
//                         write its dz; finish the previous tile (the eight
//                         slices of each sum added in a fixed order, du,
//                         ddelta, the dD and dbias accumulators).
// One barrier per tile; the staging buffers and the slices alternate between
// two LDS buffers by tile parity (159,744 bytes in all).  The arithmetic and
// its order are those of scan_bwd_kernel, and the outputs agree bit for bit
// with that kernel's except dbias (the compiler contracts a multiply and an
// add of its accumulator differently), dB/dC (the channel sums run in another
// order) and dz (silu'(z) is formed from silu(z) here, s + z s (1 - s), and as
// s (1 + z (1 - s)) there).  Three waves per SIMD need at most 168
// VGPRs: the producers keep u as loaded and softplus'(x) for a tile's finish
// and read delta and dout back from the staging buffer before overwriting it.
constexpr int kBwsRing = 2;  // producer register ring of raw rows, in tiles (a tile takes microseconds)
constexpr int kCacheNTb = 2;  // cache-policy bit NT (nontemporal) of a buffer access

// LDS slot of column q of channel row r in the role-split backward: r ^
// bws_swz(q).  The producers' 8-lane groups of a 128-bit access (rows r, r+1
// x columns 0..3) then touch 8 distinct 16-byte bank groups; the consumers'
// whole-column accesses are permutations of 64 consecutive float4s.
__device__ __forceinline__ constexpr int bws_swz(int q) { return 2 * q + 8 * (q & 1); }

template <typename T>
struct BwsRows {  // one tile's raw loads of a producer lane, as loaded
  typename Raw4<T>::type u, d, dy, z, y;
  uint32_t B, C;  // element bits
};

template <typename T, bool kHasZ, bool kAligned>
__global__ __launch_bounds__(kWsThreads) void scan_bwd_ws_kernel(
    const ScanDims p, const T* __restrict__ u, const T* __restrict__ dl,
    const float* __restrict__ Ap, const T* __restrict__ Bp, const T* __restrict__ Cp,
    const float* __restrict__ Dp, const float* __restrict__ biasp,
    const float* __restrict__ h_init, const int64_t* __restrict__ length,
    const T* __restrict__ zp, const T* __restrict__ yup, const float* __restrict__ h_chunks,
    const T* __restrict__ dyp, const float* __restrict__ dh_last, T* __restrict__ dup,
    T* __restrict__ ddp, T* __restrict__ dzp, float* __restrict__ dh_init,
    float* __restrict__ ws_bc, float* __restrict__ ws_A, float* __restrict__ ws_D,
    float* __restrict__ ws_bias, void* __restrict__ dummy, const float* __restrict__ seg_g,
    const float* __restrict__ seg_dt) {
  constexpr int kT4 = kTileB / 4;  // 4-step columns per tile
  static_assert(kTileB == kChunk, "one saved state per backward tile");
  static_assert(kWsProd * 64 == kBlockCh * kT4, "one producer lane per (row, column)");
  static_assert(2 * 2 * kWsCons * kTileB == 2 * 64 * kWsProd, "two B/C elements per producer lane");

  __shared__ float4 sSt[2][3][kT4][kBlockCh];     // [parity][delta | delta*u | dout][column][row]
  __shared__ float sBlk[2][kWsCons][kT4][16];     // [parity][pair][block][(step, state, B|C)]
  __shared__ float4 sGB[2][kWsCons][kT4][kBlockCh];  // per-wave sum_n G B
  __shared__ float4 sDD[2][kWsCons][kT4][kBlockCh];  // per-wave sum_n A G a h_{t-1}

  const int lane = threadIdx.x & 63;
  const int w = wave_id_uniform();
  const int b = blockIdx.y;
  const int blk = blockIdx.x;
  const int d0 = blk * kBlockCh;
  const int L = p.seqlen, Dm = p.dim, N = p.nstate;
  const int seg = blockIdx.z;
  const int ntiles_all = (L + kTileB - 1) / kTileB;
  const int tile_beg = seg * (p.seg_len / kTileB);
  const int tile_end = min(ntiles_all, tile_beg + p.seg_len / kTileB);
  const int nt = tile_end - tile_beg;  // tiles of this segment, walked from the end
  const int nbar = 1 + 4 * ((nt + 3) / 4);  // barriers of both roles
  const size_t srow = (size_t)seg * p.batch + b;
  const size_t rb = (size_t)b * Dm;

  if (w < kWsCons) {
    // ------------------------------------------------ consumer: the recurrences
    const int ch = d0 + lane;
    const bool ch_ok = ch < Dm;
    const int chc = min(ch, Dm - 1);
    const int Lp = bc_part_len(L);  // partial rows padded to whole tiles
    const size_t nBC = (size_t)p.batch * N * Lp;
    float gam[2], dA[2], Av[2], A2[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int n = 2 * w + s;
      const bool ok = ch_ok && n < N;
      dA[s] = 0.0f;
      Av[s] = ok ? Ap[(size_t)ch * N + n] : 0.0f;
      A2[s] = Av[s] * kLog2e;
      // carry in from the later segments, last first:
      // gamma <- gamma_seg + exp(A sum dt) gamma (their summaries, zero carry-in)
      // (summary row k: sub-segment k + sub_k of seg_len / sub_k steps)
      float q = (ok && dh_last) ? dh_last[(rb + ch) * N + n] : 0.0f;
      if (ok)
        q = fold_carry(q, A2[s], seg_dt, seg_g, (p.nseg - 1) * p.sub_k - 1, -1,
                       (p.nseg - 1 - seg) * p.sub_k, p.batch, b, Dm, N, n, ch);
      gam[s] = q;
    }
    // The state the forward saved before tile t: h_init (or zero) before
    // tile 0, else through a buffer range over the batch row's saved rows
    // (the launch keeps them below 2^31 bytes), the lane's state row as the
    // vector offset and the tile as the scalar offset.
    const int nc0 = min(2 * w, N - 1), nc1 = min(2 * w + 1, N - 1);
    const size_t hrow = (size_t)N * p.hs * Dm;  // floats per saved slot
    const auto h_rsrc = raw_rsrc(const_cast<float*>(h_chunks) + (size_t)b * p.nchunks * hrow,
                                 (uint32_t)((size_t)p.nchunks * hrow * sizeof(float)));
    const uint32_t hv0 = (uint32_t)(((size_t)nc0 * p.hs * Dm + chc) * sizeof(float));
    const uint32_t hv1 = (uint32_t)(((size_t)nc1 * p.hs * Dm + chc) * sizeof(float));
    const float hi0 = h_init ? h_init[(rb + chc) * N + nc0] : 0.0f;
    const float hi1 = h_init ? h_init[(rb + chc) * N + nc1] : 0.0f;
    // (the loads are unconditional, from slot 0 for tile 0, and the choice is
    // made where the state is used: a load inside a branch is waited for at
    // the branch's end)
    // (nontemporal loads: each saved state is read once, in whole 256-byte
    // runs, so it need not displace the input lines that serve several tiles)
    auto saved_state = [&](int tile, float (&r)[2]) {
      const int so = (int)((size_t)max(tile - 1, 0) * hrow * sizeof(float));
      r[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(h_rsrc, (int)hv0, so, kCacheNTb));
      r[1] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(h_rsrc, (int)hv1, so, kCacheNTb));
    };
    float hcn[2];
    saved_state(tile_end - 1, hcn);
    // the value of lane l after the reduction of two blocks (block of the
    // pair, kind, state, step)
    const int vi = reduce32_index(lane);
    const int rsel = vi >> 4, rkind = (vi >> 3) & 1, rs = (vi >> 2) & 1, rj = vi & 3;
    const int rn = 2 * w + rs;
    // the partials go through a buffer range over all of them (the launch
    // keeps them below 2^31 bytes): the lane's row and step as the vector
    // offset, the tile's first step as the scalar offset, the block as the
    // immediate; a state past N gets an offset past the range
    const auto bc_rsrc = raw_rsrc(ws_bc, (uint32_t)(2 * (size_t)p.nblk * nBC * sizeof(float)));
    // (the offset of the pair's second block, jq - 1; the first block adds 16
    // bytes, 4 steps, so that no offset is negative)
    const uint32_t bc_off =
        rn < N ? (uint32_t)((((size_t)rkind * p.nblk + blk) * nBC + ((size_t)b * N + rn) * Lp + rj) *
                            sizeof(float)) + 16u * (1 - rsel)
               : kOffDrop;
    const bool hc_ok0 = ch_ok && 2 * w < N, hc_ok1 = ch_ok && 2 * w + 1 < N;

    // One iteration per barrier; the staging parity is a template constant
    // (the loop runs iterations in pairs), so every LDS address is a
    // per-lane base plus an immediate.
    auto iteration = [&](int i, auto parity) {
      constexpr int buf = decltype(parity)::value;
      __syncthreads();
      if (i >= nt) return;
      const int tile = tile_end - 1 - i;
      const int t0 = tile * kTileB;
      float hc[2];
      hc[0] = tile > 0 ? (hc_ok0 ? hcn[0] : 0.0f) : hi0;
      hc[1] = tile > 0 ? (hc_ok1 ? hcn[1] : 0.0f) : hi1;
      saved_state(max(tile - 1, tile_beg), hcn);  // the next tile's (re-read at the last)

      float a[2][kChunk], H[2][kChunk];
      StepVals X, Y;
      float bcg[kT4];  // block registers of the wave's pair: lane l holds value l & 15
#pragma unroll
      for (int jq = 0; jq < kT4; ++jq) bcg[jq] = sBlk[buf][w][jq][lane & 15];
      auto put4 = [&](float4 (&slice)[kT4][kBlockCh], int q, const float (&v)[4]) {
        slice[q][lane ^ bws_swz(q)] = make_float4(v[0], v[1], v[2], v[3]);
      };
      auto fwd = [&](int jq, const StepVals& sv) {
        float y[4];  // unused here (the forward saved the output)
        bwd_recompute_block(jq, sv, bcg[jq], A2, hc, a, H, y);
      };
      // the reverse of block jq; its 16 dB/dC terms go to vals[16 * half ..]
      auto rev = [&](int jq, const StepVals& sv, float (&vals)[32], int half) {
        float gB[4], gD[4], v16[16];
        bwd_reverse_block(jq, sv, bcg[jq], Av, A2, hc, a, H, gam, dA, v16, gB, gD);
        put4(sGB[buf][w], jq, gB);
        put4(sDD[buf][w], jq, gD);
#pragma unroll
        for (int k = 0; k < 16; ++k) vals[16 * half + k] = v16[k];
      };
      // sum over the 64 channels of blocks jq and jq - 1 together
      auto reduce_store = [&](int jq, float (&vals)[32], auto old) {
        wave_reduce32<decltype(old)::value>(vals, lane);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(vals[0]), bc_rsrc,
                                              (int)(bc_off + 16u * (jq - 1)), t0 * 4, 0);
      };
      auto ld = [&](int jq, StepVals& sv, bool with_dout) {
        const int li = lane ^ bws_swz(jq);
        sv.dl = sSt[buf][0][jq][li];
        sv.du = sSt[buf][1][jq][li];
        if (with_dout) sv.dout = sSt[buf][2][jq][li];
      };
      // fixed schedule F0 F1 F2 F3 R3 R2 R1 R0 (recompute, then reverse)
      ld(0, X, false); fwd(0, X);
      ld(1, Y, false); fwd(1, Y);
      ld(2, X, false); fwd(2, X);
      ld(3, Y, true);  fwd(3, Y);
      // the reverse re-reads the block registers: hide their values from
      // the recompute's, so each DPP broadcast folds into its own multiply
      // (shared, it is materialised with an extra v_mov_dpp and a register)
#pragma unroll
      for (int jq = 0; jq < kT4; ++jq) asm volatile("" : "+v"(bcg[jq]));
      // blocks 3 and 2 are reduced after block 1's reverse, so their terms
      // are not fresh VALU results at the folds
      float v32[32], w32[32];
      // X still holds block 2's delta and delta*u: read its dout only, and
      // block 1's values a block ahead of their use
      X.dout = sSt[buf][2][2][lane ^ bws_swz(2)];
      StepVals Z;
      ld(1, Z, true);
      rev(3, Y, v32, 0);
      rev(2, X, v32, 1);
      ld(0, Y, true);
      rev(1, Z, w32, 0);
      reduce_store(3, v32, std::true_type{});
      rev(0, Y, w32, 1);
      reduce_store(1, w32, std::false_type{});
    };
    // nbar - 1 is a multiple of 4: iteration 0, then pairs of parity 1, 0
    iteration(0, std::integral_constant<int, 0>{});
    for (int i = 1; i < nbar; i += 2) {
      iteration(i, std::integral_constant<int, 1>{});
      iteration(i + 1, std::integral_constant<int, 0>{});
    }
    // per-row partials
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int n = 2 * w + s;
      if (ch_ok && n < N) {
        ws_A[(srow * Dm + ch) * N + n] = dA[s];
        if (dh_init && seg == 0) dh_init[(rb + ch) * N + n] = gam[s];
      }
    }
    return;
  }

  // ------------------------------------------------ producer: staging and per-position gradients
  const int pt = (w - kWsCons) * 64 + lane;
  const int row = pt / kT4;
  const int q = pt % kT4;
  const int sw = row ^ bws_swz(q);
  const int pch = d0 + row;
  const bool pch_ok = pch < Dm;
  const int chc = min(pch, Dm - 1);
  const float Dv = (pch_ok && Dp) ? Dp[pch] : 0.0f;
  const float Bias = (pch_ok && biasp) ? biasp[pch] : 0.0f;
  const T* __restrict__ u_row = u + (rb + chc) * L;
  const T* __restrict__ d_row = dl + (rb + chc) * L;
  const T* __restrict__ dy_row = dyp + (rb + chc) * L;
  const T* __restrict__ z_row = kHasZ ? zp + (rb + chc) * L : u_row;
  const T* __restrict__ y_row = kHasZ ? yup + (rb + chc) * L : u_row;
  int vlo, vhi;
  valid_window(length, p.pad_right, b, L, vlo, vhi);
  const bool softplus = p.softplus != 0;
  // B/C staging: lane pt -> state n = (pt / 16) % 16 and step pt % 16 of B
  // (first element) and of C (second)
  const int bc_n = (pt / kTileB) % (2 * kWsCons);
  const int bc_j = pt % kTileB;
  const bool bc_ok = bc_n < N;
  const size_t bc_row = (size_t)b * p.bc_bstride + (size_t)min(bc_n, N - 1) * L;
  const T* __restrict__ B_row = Bp + bc_row;
  const T* __restrict__ C_row = Cp + bc_row;
  const int bc_slot = (bc_j & 3) * 4 + (bc_n & 1) * 2;  // B; C at + 1
  // tile index of iteration i (clamped to the segment: tiles past it are
  // staged from valid rows and never used)
  auto tile_of = [&](int i) { return max(tile_end - 1 - i, tile_beg); };
  // Output buffers of this wave's 16 channel rows (aligned path; the launch
  // keeps 16 * L * sizeof(T) < 2^31): a masked lane, a step past L or a tile
  // past the segment gets an offset outside the range and the store is dropped.
  const int wrow0 = d0 + (w - kWsCons) * (kBlockCh / kWsProd);
  const uint32_t wbytes =
      (uint32_t)(max(0, min(kBlockCh / kWsProd, Dm - wrow0)) * (size_t)L * sizeof(T));
  const auto du_rsrc = raw_rsrc(dup + ((size_t)rb + wrow0) * L, wbytes);
  const auto dd_rsrc = raw_rsrc(ddp + ((size_t)rb + wrow0) * L, wbytes);
  const auto dz_rsrc = raw_rsrc(kHasZ ? dzp + ((size_t)rb + wrow0) * L : dup, kHasZ ? wbytes : 0u);
  const uint32_t row_off = (uint32_t)((row % (kBlockCh / kWsProd)) * (size_t)L * sizeof(T));

  // The aligned path's loads go through buffer ranges over the same 16 rows,
  // and over the batch row's B and C rows, at 32-bit offsets (no 64-bit
  // address arithmetic per tile).  The step is clamped into the row as on the
  // pointer path; a row past the last channel reads zero.
  const auto u_ld = raw_rsrc(const_cast<T*>(u) + ((size_t)rb + wrow0) * L, wbytes);
  const auto d_ld = raw_rsrc(const_cast<T*>(dl) + ((size_t)rb + wrow0) * L, wbytes);
  const auto dy_ld = raw_rsrc(const_cast<T*>(dyp) + ((size_t)rb + wrow0) * L, wbytes);
  const auto z_ld = raw_rsrc(kHasZ ? const_cast<T*>(zp) + ((size_t)rb + wrow0) * L : const_cast<T*>(u),
                             kHasZ ? wbytes : 0u);
  const auto y_ld = raw_rsrc(kHasZ ? const_cast<T*>(yup) + ((size_t)rb + wrow0) * L : const_cast<T*>(u),
                             kHasZ ? wbytes : 0u);
  const uint32_t bc_bytes = (uint32_t)((size_t)N * L * sizeof(T));
  const auto B_ld = raw_rsrc(const_cast<T*>(Bp) + (size_t)b * p.bc_bstride, bc_bytes);
  const auto C_ld = raw_rsrc(const_cast<T*>(Cp) + (size_t)b * p.bc_bstride, bc_bytes);
  const uint32_t bc_row_off = (uint32_t)((size_t)min(bc_n, N - 1) * L * sizeof(T));

  auto issue = [&](BwsRows<T>& r, int i) {
    if constexpr (kAligned) {
      const int t0 = tile_of(i) * kTileB;
      const uint32_t off = row_off + (uint32_t)min(t0 + 4 * q, L - 4) * sizeof(T);
      r.u = buffer_load_raw4<T>(u_ld, off);
      r.d = buffer_load_raw4<T>(d_ld, off);
      r.dy = buffer_load_raw4<T>(dy_ld, off);
      if constexpr (kHasZ) {
        r.z = buffer_load_raw4<T>(z_ld, off);
        r.y = buffer_load_raw4<T>(y_ld, off);
      } else {
        r.z = r.y = typename Raw4<T>::type{};
      }
      const uint32_t boff = bc_row_off + (uint32_t)min(t0 + bc_j, L - 1) * sizeof(T);
      r.B = buffer_load_bits1<T>(B_ld, boff);
      r.C = buffer_load_bits1<T>(C_ld, boff);
      return;
    }
    const int t = tile_of(i) * kTileB + 4 * q;
    r.u = load_raw4_nb<T, kAligned>(u_row, t, L, pch_ok);
    r.d = load_raw4_nb<T, kAligned>(d_row, t, L, pch_ok);
    r.dy = load_raw4_nb<T, kAligned>(dy_row, t, L, pch_ok);
    if constexpr (kHasZ) {
      r.z = load_raw4_nb<T, kAligned>(z_row, t, L, pch_ok);
      r.y = load_raw4_nb<T, kAligned>(y_row, t, L, pch_ok);
    } else {
      r.z = r.y = typename Raw4<T>::type{};
    }
    const int tb = min(tile_of(i) * kTileB + bc_j, L - 1);
    r.B = elem_bits(B_row[tb]);
    r.C = elem_bits(C_row[tb]);
  };

  // What a tile's finish needs from its staging besides delta and dout (read
  // back from the staging buffer before the next staging overwrites it): u as
  // loaded and softplus'(x) (zero where masked).
  struct Kept {
    typename Raw4<T>::type u;
    float sg[4];
  };

  // stage iteration i's tile into buffer i & 1 and write its dz
  auto stage = [&](const BwsRows<T>& r, int i, Kept& k) {
    const int tile = tile_of(i);
    const int t0 = tile * kTileB;
    const int t = t0 + 4 * q;
    const int sb = i & 1;
    float uv[4], dv[4], dyv[4];
    decode4(r.u, uv);
    decode4(r.d, dv);
    decode4(r.dy, dyv);
    float de[4], du[4], dov[4], dzo[4], dym[4];
    // (softplus is uniform: a branch, not a select after both forms)
    if (softplus) {
#pragma unroll
      for (int j = 0; j < 4; ++j) softplus_and_grad_u(dv[j] + Bias, de[j], k.sg[j]);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        de[j] = dv[j] + Bias;
        k.sg[j] = 1.0f;
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) dym[j] = dyv[j];
    // Steps outside the valid window are masked on the tiles that hold any (at
    // most two per row).  Rows past the last channel read zero on the aligned
    // path (outside the wave's buffer range), so their delta * u and dout, and
    // every term those feed, are zero unmasked; the pointer path reads the
    // clamped channel there and masks them on every tile.
    if (!kAligned || !(t0 >= vlo && t0 + kTileB <= vhi)) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t keep = (pch_ok & (t + j >= vlo) & (t + j < vhi)) ? ~0u : 0u;
        de[j] = __uint_as_float(__float_as_uint(de[j]) & keep);
        k.sg[j] = __uint_as_float(__float_as_uint(k.sg[j]) & keep);
        dym[j] = __uint_as_float(__float_as_uint(dym[j]) & keep);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      du[j] = de[j] * uv[j];
      if constexpr (kHasZ) {
        float zv[4], yv[4];
        decode4(r.z, zv);
        decode4(r.y, yv);
        // silu(z) = z s and silu'(z) = s + z s (1 - s), s = sigmoid(z)
        const float sz = sigmoidf_fast(zv[j]);
        const float zs = zv[j] * sz;
        dov[j] = dym[j] * zs;
        dzo[j] = dyv[j] * yv[j] * fmaf(zs, 1.0f - sz, sz);  // every position
      } else {
        dov[j] = dym[j];
        dzo[j] = 0.0f;
      }
    }
    k.u = r.u;
    sSt[sb][0][q][sw] = make_float4(de[0], de[1], de[2], de[3]);
    sSt[sb][1][q][sw] = make_float4(du[0], du[1], du[2], du[3]);
    sSt[sb][2][q][sw] = make_float4(dov[0], dov[1], dov[2], dov[3]);
    float* const blk_dst = &sBlk[sb][bc_n >> 1][bc_j >> 2][bc_slot];
    blk_dst[0] = bc_ok ? bits_to_f32<T>(r.B) : 0.0f;
    blk_dst[1] = bc_ok ? bits_to_f32<T>(r.C) : 0.0f;
    // a tile past the segment (i >= nt) writes nothing
    const bool st_ok = pch_ok && i < nt;
    if constexpr (kHasZ) {
      if constexpr (kAligned)
        buffer_store4<T>(dz_rsrc, (i < nt && t < L) ? row_off + (uint32_t)t * sizeof(T) : kOffDrop,
                         dzo);
      else
        store4_nb<T, kAligned>(dzp + (rb + pch) * L, t, L, st_ok, dummy, dzo);
    }
  };

  float accD = 0.0f, accB = 0.0f;
  // finish iteration i's tile: slices of parity i & 1
  auto finish = [&](int i, const Kept& k) {
    const int tile = tile_of(i);
    const int t = tile * kTileB + 4 * q;
    const int sb = i & 1;
    float4 gb = sGB[sb][0][q][sw], gd = sDD[sb][0][q][sw];
#pragma unroll
    for (int ww = 1; ww < kWsCons; ++ww) {
      const float4 q1 = sGB[sb][ww][q][sw];
      gb.x += q1.x; gb.y += q1.y; gb.z += q1.z; gb.w += q1.w;
    }
#pragma unroll
    for (int ww = 1; ww < kWsCons; ++ww) {
      const float4 q2 = sDD[sb][ww][q][sw];
      gd.x += q2.x; gd.y += q2.y; gd.z += q2.z; gd.w += q2.w;
    }
    const float gbv[4] = {gb.x, gb.y, gb.z, gb.w};
    const float gdv[4] = {gd.x, gd.y, gd.z, gd.w};
    float de[4], dov[4], uu[4];
    f4_to(sSt[sb][0][q][sw], de);
    f4_to(sSt[sb][2][q][sw], dov);
    decode4(k.u, uu);
    float duo[4], ddo[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      duo[j] = fmaf(Dv, dov[j], de[j] * gbv[j]);
      ddo[j] = fmaf(uu[j], gbv[j], gdv[j]) * k.sg[j];  // sg is 0 at padded steps
    }
    const bool ok = i < nt;
    if (ok) {  // no memory operations inside
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        accD = fmaf(dov[j], uu[j], accD);  // dov is 0 at padded steps
        accB += ddo[j];
      }
    }
    if constexpr (kAligned) {
      const uint32_t off = (ok && t < L) ? row_off + (uint32_t)t * sizeof(T) : kOffDrop;
      buffer_store4<T>(du_rsrc, off, duo);
      buffer_store4<T>(dd_rsrc, off, ddo);
    } else {
      store4_nb<T, kAligned>(dup + (rb + pch) * L, t, L, ok && pch_ok, dummy, duo);
      store4_nb<T, kAligned>(ddp + (rb + pch) * L, t, L, ok && pch_ok, dummy, ddo);
    }
  };

  // Iteration i after barrier i: finish tile i-1 (its slices were written
  // during iteration i-1), then stage tile i+1 into the buffer tile i-1 used.
  // Raw rows travel in a ring of kBwsRing tiles (tile k's loads are issued
  // when tile k - kBwsRing is staged); what a finish needs rides in a ring of
  // 4 tiles (staged at iteration k - 1, finished at k + 1).  Iterations
  // 1 .. 4m run in unrolled groups of four with no conditions around memory
  // operations, so the compiler's waits for the ring's loads count exactly.
  BwsRows<T> rows[kBwsRing];
  Kept kept[4];
#pragma unroll
  for (int k2 = 0; k2 < kBwsRing; ++k2) issue(rows[k2], k2);
  stage(rows[0], 0, kept[0]);
  issue(rows[0], kBwsRing);
  __syncthreads();  // iteration 0
  stage(rows[1], 1, kept[1]);
  issue(rows[1], kBwsRing + 1);
  for (int i0 = 1; i0 < nbar; i0 += 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = i0 + j;  // (i + 1) % 4 == (j + 2) % 4, (i - 1) % 4 == j
      __syncthreads();
      finish(i - 1, kept[j]);
      stage(rows[(j + 2) % kBwsRing], i + 1, kept[(j + 2) & 3]);
      issue(rows[(j + 2) % kBwsRing], i + 1 + kBwsRing);
    }
  }
  // dD from dout * u, dbias from ddelta: the 4 lanes of a row are
  // consecutive
  const float sd = group_sum<kT4>(accD);
  const float sbias = group_sum<kT4>(accB);
  if (pch_ok && q == 0) {
    ws_D[srow * Dm + pch] = sd;
    ws_bias[srow * Dm + pch] = sbias;
  }
}

// ---------------------------------------------------------------- state chunks

// After the kPart backward: per (batch row b, channel d), the per-position
// gradients from the state chunks' sums (added in chunk order):
//   gb = sum_n G B, gd = sum_n A G a h_{t-1};
//   du = D * dout + delta * gb;  ddelta = softplus'(x) * (u * gb + gd);
// with dout the masked (and gated) upstream gradient as in the main kernel,
// and the row's dD = sum_t dout u and dbias = sum_t ddelta written as the
// (segment 0, b) partial rows (the other segments' rows are zeroed).
template <typename T, bool kHasZ>
__global__ __launch_bounds__(256) void scan_bwd_combine_kernel(
    const ScanDims p, const int nsc, const T* __restrict__ u, const T* __restrict__ dl,
    const T* __restrict__ dyp, const T* __restrict__ zp, const float* __restrict__ Dp,
    const float* __restrict__ biasp, const int64_t* __restrict__ length,
    const float* __restrict__ ws_gb, const float* __restrict__ ws_gd, T* __restrict__ dup,
    T* __restrict__ ddp, float* __restrict__ ws_D, float* __restrict__ ws_bias) {
  __shared__ float red[2][256 / 64];
  const int d = blockIdx.x, b = blockIdx.y;
  const int L = p.seqlen, Dm = p.dim;
  const size_t row = ((size_t)b * Dm + d) * L;
  const size_t cstride = (size_t)p.batch * Dm * L;
  int vlo, vhi;
  valid_window(length, p.pad_right, b, L, vlo, vhi);
  const float Dv = Dp ? Dp[d] : 0.0f;
  const float Bias = biasp ? biasp[d] : 0.0f;
  const bool softplus = p.softplus != 0;
  float accD = 0.0f, accB = 0.0f;
  for (int t = threadIdx.x; t < L; t += blockDim.x) {
    const bool valid = t >= vlo && t < vhi;
    const float uu = Elem<T>::load1(u + row + t);
    const float x = Elem<T>::load1(dl + row + t) + Bias;
    float dt = x, sg = 1.0f;
    if (softplus) softplus_and_grad_t20(x, dt, sg);
    float dout = valid ? Elem<T>::load1(dyp + row + t) : 0.0f;
    if constexpr (kHasZ) {
      const float zz = Elem<T>::load1(zp + row + t);
      dout *= zz * sigmoidf_fast(zz);
    }
    float gb = 0.0f, gd = 0.0f;
    for (int c = 0; c < nsc; ++c) {
      gb += ws_gb[c * cstride + row + t];
      gd += ws_gd[c * cstride + row + t];
    }
    const float de = valid ? dt : 0.0f;
    const float du = fmaf(Dv, dout, de * gb);
    const float dd = valid ? fmaf(uu, gb, gd) * sg : 0.0f;
    accD = fmaf(dout, uu, accD);
    accB += dd;
    Elem<T>::store1(dup + row + t, du);
    Elem<T>::store1(ddp + row + t, dd);
  }
  accD = group_sum<64>(accD);
  accB = group_sum<64>(accB);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[0][w] = accD;
    red[1][w] = accB;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float sd = 0.0f, sb = 0.0f;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) {
      sd += red[0][i];
      sb += red[1][i];
    }
    for (int s = 0; s < p.nseg; ++s) {
      const size_t r = ((size_t)s * p.batch + b) * Dm + d;
      ws_D[r] = s == 0 ? sd : 0.0f;
      ws_bias[r] = s == 0 ? sb : 0.0f;
    }
  }
}

// ---------------------------------------------------------------- segment summaries

// For segment s = blockIdx.z + 1 (segments 1 .. nseg-1) of batch row b and 64
// channels: the adjoint carry the segment hands to the one before it when its
// own carry-in is zero, gamma_seg (the reverse recurrence G_t = gamma_t +
// dout_t C_t, gamma_{t-1} = a_t G_t run from the segment's last step down to
// its first), and the segment's summed step size.  With a carry-in q the
// segment hands on gamma_seg + exp(A sum dt) q, which the main backward folds
// from the last segment down.  dout is masked and gated exactly as in the main
// kernel.  Tiles of 32 steps walked backwards; phase A stages delta and the
// effective dout (double-buffered by tile parity: one barrier per tile) and
// the tile's (C0, C1) per state pair.
template <typename T, int kSG, bool kHasZ, bool kAligned>
__global__ __launch_bounds__(kThreads) void scan_bwd_segsum_kernel(
    const ScanDims p, const T* __restrict__ dl, const T* __restrict__ dyp,
    const T* __restrict__ zp, const float* __restrict__ Ap, const float* __restrict__ bc,
    const float* __restrict__ biasp, const int64_t* __restrict__ length,
    float* __restrict__ seg_g, float* __restrict__ seg_dt) {
  using R4 = typename Raw4<T>::type;
  constexpr int kTS = 32;  // steps per tile
  constexpr int kT4 = kTS / 4;
  static_assert(kBlockCh * kT4 == kThreads, "one 4-step row piece per thread");
  __shared__ float4 sDelta[2][kT4][kBlockCh];
  __shared__ float4 sDo[2][kT4][kBlockCh];
  __shared__ float4 sC[2][kWaves][kTS / 2];  // (C0, C1) of steps 2i, 2i+1 per pair

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = wave_id_uniform();
  const int b = blockIdx.y;
  const int d0 = blockIdx.x * kBlockCh;
  // blockIdx.z = (state chunk sc) * (nseg - 1) + segment - 1; sc > 0 only
  // for the state chunks of the kPart backward (states n0 .. n0 + 63)
  const int seg = (int)blockIdx.z % (p.nseg - 1) + 1;
  const int n0 = (int)blockIdx.z / (p.nseg - 1) * (2 * kWaves * kSG);
  const int L = p.seqlen, Dm = p.dim, N = p.nstate;
  const int Tbeg = seg * p.seg_len;
  const int Lend = min(L, Tbeg + p.seg_len);
  const int npair = bc_pairs(N);
  const int Lp = bc_row_len(L);
  const size_t rb = (size_t)b * Dm;
  int vlo, vhi;
  valid_window(length, p.pad_right, b, L, vlo, vhi);

  const int ch = d0 + lane;
  const bool ch_ok = ch < Dm;
  float gam[kSG][2], A2[kSG][2];
#pragma unroll
  for (int g = 0; g < kSG; ++g)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int n = n0 + (g * kWaves + w) * 2 + s;
      A2[g][s] = (ch_ok && n < N) ? Ap[(size_t)ch * N + n] * kLog2e : 0.0f;
      gam[g][s] = 0.0f;
    }

  const int a_row = tid / kT4;
  const int a_q = tid % kT4;
  const int a_col = a_q * 4;
  // the forward's column swizzle (8 columns of 4 steps)
  const int a_sw = a_row ^ (a_q | ((a_q & 1) << 3));
  const int a_ch = d0 + a_row;
  const bool a_ok = a_ch < Dm;
  const float Bias = (a_ok && biasp) ? biasp[a_ch] : 0.0f;
  const int a_chc = min(a_ch, Dm - 1);
  const T* __restrict__ d_row = dl + (rb + a_chc) * L;
  const T* __restrict__ y_row = dyp + (rb + a_chc) * L;
  const T* __restrict__ z_row = kHasZ ? zp + (rb + a_chc) * L : y_row;
  const bool softplus = p.softplus != 0;
  const float4* __restrict__ bc4 = reinterpret_cast<const float4*>(bc);
  const int c_G = (tid / kTS) % kWaves;
  const int c_t = tid % kTS;
  auto load_c = [&](int T0) {
    const int t = min(T0 + c_t, Lp - 1);
    return bc4[((size_t)b * npair + c_G) * Lp + t];
  };
  const int Tlast = Tbeg + (Lend - 1 - Tbeg) / kTS * kTS;
  float dtsum = 0.0f;

  R4 qd = load_raw4_nb<T, kAligned>(d_row, Tlast + a_col, L, a_ok);
  R4 qy = load_raw4_nb<T, kAligned>(y_row, Tlast + a_col, L, a_ok);
  R4 qz = kHasZ ? load_raw4_nb<T, kAligned>(z_row, Tlast + a_col, L, a_ok) : R4{};
  float4 qc = kSG == 1 ? load_c(Tlast) : make_float4(0.f, 0.f, 0.f, 0.f);
  int buf = 0;
  for (int T0 = Tlast; T0 >= Tbeg; T0 -= kTS) {
    {
      float dv[4], yv[4], zv[4], de[4], dov[4];
      decode4(qd, dv);
      decode4(qy, yv);
      if constexpr (kHasZ) decode4(qz, zv);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tt = T0 + a_col + j;
        const bool valid = a_ok && tt >= vlo && tt < vhi && tt < Lend;
        const float x = dv[j] + Bias;
        const float dt = softplus ? softplus_t20(x) : x;
        de[j] = valid ? dt : 0.0f;
        const float dym = valid ? yv[j] : 0.0f;
        if constexpr (kHasZ) dov[j] = dym * (zv[j] * sigmoidf_fast(zv[j]));
        else dov[j] = dym;
        dtsum += de[j];
      }
      sDelta[buf][a_q][a_sw] = make_float4(de[0], de[1], de[2], de[3]);
      sDo[buf][a_q][a_sw] = make_float4(dov[0], dov[1], dov[2], dov[3]);
      if (kSG == 1 && tid < kWaves * kTS) {
        float* row = reinterpret_cast<float*>(&sC[buf][c_G][0]);
        row[2 * c_t] = qc.y;
        row[2 * c_t + 1] = qc.w;
      }
    }
    // the previous tile in time (the first tile re-reads itself)
    const int Tn = max(T0 - kTS, Tbeg);
    qd = load_raw4_nb<T, kAligned>(d_row, Tn + a_col, L, a_ok);
    qy = load_raw4_nb<T, kAligned>(y_row, Tn + a_col, L, a_ok);
    if constexpr (kHasZ) qz = load_raw4_nb<T, kAligned>(z_row, Tn + a_col, L, a_ok);
    if constexpr (kSG == 1) qc = load_c(Tn);
    __syncthreads();
    // steps past Lend hold zeros (identity steps), so whole tiles are walked
    if constexpr (kSG == 1) {
      const float4* __restrict__ cro = sC[buf][w];
#pragma unroll
      for (int k = kT4 - 1; k >= 0; --k) {
        const float4 dl4 = sDelta[buf][k][lane ^ (k | ((k & 1) << 3))];
        const float4 do4 = sDo[buf][k][lane ^ (k | ((k & 1) << 3))];
        const float4 c01 = cro[2 * k], c23 = cro[2 * k + 1];
        const float dlv[4] = {dl4.x, dl4.y, dl4.z, dl4.w};
        const float dov[4] = {do4.x, do4.y, do4.z, do4.w};
        const float c0[4] = {c01.x, c01.z, c23.x, c23.z};
        const float c1[4] = {c01.y, c01.w, c23.y, c23.w};
#pragma unroll
        for (int j = 3; j >= 0; --j) {
          gam[0][0] = fast_exp2(dlv[j] * A2[0][0]) * fmaf(dov[j], c0[j], gam[0][0]);
          gam[0][1] = fast_exp2(dlv[j] * A2[0][1]) * fmaf(dov[j], c1[j], gam[0][1]);
        }
      }
    } else {
      for (int k = kT4 - 1; k >= 0; --k) {
        const float4 dl4 = sDelta[buf][k][lane ^ (k | ((k & 1) << 3))];
        const float4 do4 = sDo[buf][k][lane ^ (k | ((k & 1) << 3))];
        const float dlv[4] = {dl4.x, dl4.y, dl4.z, dl4.w};
        const float dov[4] = {do4.x, do4.y, do4.z, do4.w};
        const int tb = min(T0 + 4 * k, Lp - 4);
#pragma unroll
        for (int g = 0; g < kSG; ++g) {
          const int G = n0 / 2 + g * kWaves + w;
          if (G < npair) {
            const float4* __restrict__ q = bc4 + ((size_t)b * npair + G) * Lp + tb;
#pragma unroll
            for (int j = 3; j >= 0; --j) {
              const float4 v = q[j];  // (B0, C0, B1, C1), wave-uniform
              gam[g][0] = fast_exp2(dlv[j] * A2[g][0]) * fmaf(dov[j], v.y, gam[g][0]);
              gam[g][1] = fast_exp2(dlv[j] * A2[g][1]) * fmaf(dov[j], v.w, gam[g][1]);
            }
          }
        }
      }
    }
    buf ^= 1;
  }

  const size_t sb = (size_t)(seg - 1) * p.batch + b;
  if (ch_ok) {
#pragma unroll
    for (int g = 0; g < kSG; ++g)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int n = n0 + (g * kWaves + w) * 2 + s;
        if (n < N) seg_g[(sb * N + n) * Dm + ch] = gam[g][s];
      }
  }
#pragma unroll
  for (int m = 1; m < kT4; m <<= 1) dtsum += __shfl_xor(dtsum, m, 64);
  if (a_q == 0 && a_ok && n0 == 0) seg_dt[sb * Dm + a_ch] = dtsum;
}

// Role-split segment summaries of the backward for up to 16 states: the
// numbers scan_bwd_segsum_kernel computes, per sub-segment of seg_len / sub_k
// steps (blockIdx.z = k: global sub-segment k + sub_k, so the sub-segments
// of segments 1 .. nseg-1), with the forward's role split so that staging
// overlaps the recurrence:
//   consumer waves 0..7   lane = channel, wave w = states 2w and 2w+1: from
//                         gamma = 0 after the sub-segment's last step, down
//                         to its first, G_t = gamma_t + dout_t C_t and
//                         gamma_{t-1} = a_t G_t, reading delta, the effective
//                         dout and (C_2w, C_2w+1) from LDS;
//   producer waves 8..11  lane -> (channel row, 4-step column): stage the
//                         16-step tiles two ahead of the walk (softplus, the
//                         window mask, dout * silu(z), C), and sum the
//                         steps' delta.
// The main backward folds the summaries from the last sub-segment down to
// the first one after its segment.  A sub-segment past the sequence end has
// no tiles and leaves gamma = 0 and sum dt = 0 (the identity).
template <typename T, bool kHasZ, bool kAligned>
__global__ __launch_bounds__(kWsThreads, kAligned ? 6 : 5) void scan_bwd_segsum_ws_kernel(
    const ScanDims p, const T* __restrict__ dl, const T* __restrict__ dyp,
    const T* __restrict__ zp, const float* __restrict__ Ap, const T* __restrict__ Cp,
    const float* __restrict__ biasp, const int64_t* __restrict__ length,
    float* __restrict__ seg_g, float* __restrict__ seg_dt) {
  // raw rows in flight: 4 tiles; 2 for fp32, whose 16-byte pieces would
  // otherwise hold the producers above the registers of two workgroups per CU
  constexpr int kTile = 16, kT4 = kTile / 4, kStage = 3, kRing = sizeof(T) == 4 ? 2 : 4;
  constexpr int kRow = kBlockCh + 2;  // column length in float4s (the forward's padding)
  static_assert(kWsProd * 64 == kBlockCh * kT4, "one producer lane per (row, column)");
  static_assert(2 * kWsCons * kTile == 64 * kWsProd, "one C element per producer lane");
  __shared__ float4 sSt[kStage][2][kT4][kRow];   // [delta | effective dout][column][row]
  __shared__ float4 sC[kStage][kWsCons][kTile / 2];  // (C_2w, C_2w+1) of steps 2i, 2i+1

  const int lane = threadIdx.x & 63;
  const int w = wave_id_uniform();
  const int b = blockIdx.y;
  const int d0 = blockIdx.x * kBlockCh;
  const int L = p.seqlen, Dm = p.dim, N = p.nstate;
  int Tbeg, Lend;
  sub_range(p, (int)blockIdx.z + p.sub_k, Tbeg, Lend);
  const int ntiles = max(0, (Lend - Tbeg + kTile - 1) / kTile);
  const size_t sb = (size_t)blockIdx.z * p.batch + b;  // summary row
  // tile i of the walk starts at step tile_t(i): the last tile first
  auto tile_t = [&](int i) { return Tbeg + (ntiles - 1 - i) * kTile; };
  // as many barriers on both sides: 1 + 4 * ceil(ntiles / 4)
  const int nbar = 1 + 4 * ((ntiles + 3) / 4);

  if (w < kWsCons) {
    // ------------------------------------------------ consumer: the reverse recurrence
    const int ch = d0 + lane;
    const bool ch_ok = ch < Dm;
    float gam[2] = {0.0f, 0.0f}, A2[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int n = 2 * w + s;
      A2[s] = (ch_ok && n < N) ? Ap[(size_t)ch * N + n] * kLog2e : 0.0f;
    }
    // block k: delta and dout of steps 4k .. 4k+3, and (C0, C1) of those
    // steps as two float4s (the same address in every lane: broadcast reads)
    float4 dlb[2], dob[2], cb[2][2];
    auto read_block = [&](int buf, int k, float4& dl4, float4& do4, float4 (&c)[2]) {
      const float4* __restrict__ st = &sSt[buf][0][0][lane];
      dl4 = st[k * kRow];
      do4 = st[(kT4 + k) * kRow];
      c[0] = sC[buf][w][2 * k];
      c[1] = sC[buf][w][2 * k + 1];
    };
    int buf = 0;
    for (int i = 0; i < nbar; ++i) {
      __syncthreads();
      if (i >= ntiles) continue;
      if (i == 0) read_block(0, kT4 - 1, dlb[0], dob[0], cb[0]);
      const int nbuf = buf == kStage - 1 ? 0 : buf + 1;
      // block k - 1's LDS reads are issued before block k is computed; after
      // block 0, the next tile's last block (staged one iteration ago)
#pragma unroll
      for (int kk = 0; kk < kT4; ++kk) {
        const int c = kk & 1;
        if (kk + 1 < kT4) read_block(buf, kT4 - 2 - kk, dlb[c ^ 1], dob[c ^ 1], cb[c ^ 1]);
        else read_block(nbuf, kT4 - 1, dlb[c ^ 1], dob[c ^ 1], cb[c ^ 1]);
        const float dlv[4] = {dlb[c].x, dlb[c].y, dlb[c].z, dlb[c].w};
        const float dov[4] = {dob[c].x, dob[c].y, dob[c].z, dob[c].w};
        const float c0[4] = {cb[c][0].x, cb[c][0].z, cb[c][1].x, cb[c][1].z};
        const float c1[4] = {cb[c][0].y, cb[c][0].w, cb[c][1].y, cb[c][1].w};
#pragma unroll
        for (int j = 3; j >= 0; --j) {
          gam[0] = fast_exp2(dlv[j] * A2[0]) * fmaf(dov[j], c0[j], gam[0]);
          gam[1] = fast_exp2(dlv[j] * A2[1]) * fmaf(dov[j], c1[j], gam[1]);
        }
      }
      static_assert(kT4 % 2 == 0, "the last block of every tile in register set 0");
      buf = nbuf;
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int n = 2 * w + s;
      if (ch_ok && n < N) seg_g[(sb * N + n) * Dm + ch] = gam[s];
    }
    return;
  }

  // ------------------------------------------------ producer: staging and step sums
  const int pt = (w - kWsCons) * 64 + lane;
  const int row = pt / kT4;
  const int q = pt % kT4;
  const int pch = d0 + row;
  const bool pch_ok = pch < Dm;
  const float Bias = (pch_ok && biasp) ? biasp[pch] : 0.0f;
  const int chc = min(pch, Dm - 1);
  const size_t rb = (size_t)b * Dm;
  int vlo, vhi;
  valid_window(length, p.pad_right, b, L, vlo, vhi);
  vlo = max(vlo, Tbeg);  // steps outside the sub-segment are identity steps
  vhi = min(vhi, Lend);
  const bool softplus = p.softplus != 0;
  // C staging: producer lane pt -> (state 2G + half, step) of a tile
  const int c_half = pt / (kWsCons * kTile);
  const int c_G = (pt / kTile) % kWsCons;
  const int c_step = pt % kTile;
  const int c_n = 2 * c_G + c_half;
  const bool c_ok = c_n < N;
  const size_t c_row = (size_t)b * p.bc_bstride + (size_t)min(c_n, N - 1) * L;
  // aligned rows: buffer ranges over the wave's 16 channel rows (the launch
  // keeps 16 * L * sizeof(T) below 2^31) and over the batch row's C rows
  const int wrow0 = d0 + (w - kWsCons) * (kBlockCh / kWsProd);
  const uint32_t wbytes =
      (uint32_t)(max(0, min(kBlockCh / kWsProd, Dm - wrow0)) * (size_t)L * sizeof(T));
  const uint32_t row_off = (uint32_t)((row % (kBlockCh / kWsProd)) * (size_t)L * sizeof(T));
  const auto d_ld = raw_rsrc(const_cast<T*>(dl) + (rb + wrow0) * L, wbytes);
  const auto y_ld = raw_rsrc(const_cast<T*>(dyp) + (rb + wrow0) * L, wbytes);
  const auto z_ld = raw_rsrc(kHasZ ? const_cast<T*>(zp) + (rb + wrow0) * L : const_cast<T*>(dyp),
                             kHasZ ? wbytes : 0u);
  const auto C_ld = raw_rsrc(const_cast<T*>(Cp) + (size_t)b * p.bc_bstride,
                             (uint32_t)((size_t)N * L * sizeof(T)));
  const uint32_t c_row_off = (uint32_t)((size_t)min(c_n, N - 1) * L * sizeof(T));
  const T* __restrict__ d_row = dl + (rb + chc) * L;
  const T* __restrict__ y_row = dyp + (rb + chc) * L;
  const T* __restrict__ z_row = kHasZ ? zp + (rb + chc) * L : y_row;

  struct Rows {
    typename Raw4<T>::type d, y, z;
    uint32_t C;
  };
  // raw loads of tile i, the step clamped into the row (tiles past the walk
  // load data that is never used)
  auto issue = [&](Rows& r, int i) {
    const int t0 = max(tile_t(i), 0);
    if constexpr (kAligned) {
      const uint32_t off = row_off + (uint32_t)min(t0 + 4 * q, L - 4) * sizeof(T);
      r.d = buffer_load_raw4<T>(d_ld, off);
      r.y = buffer_load_raw4<T>(y_ld, off);
      if constexpr (kHasZ) r.z = buffer_load_raw4<T>(z_ld, off);
      else r.z = typename Raw4<T>::type{};
      r.C = buffer_load_bits1<T>(C_ld, c_row_off + (uint32_t)min(t0 + c_step, L - 1) * sizeof(T));
    } else {
      r.d = load_raw4_nb<T, kAligned>(d_row, t0 + 4 * q, L, pch_ok);
      r.y = load_raw4_nb<T, kAligned>(y_row, t0 + 4 * q, L, pch_ok);
      if constexpr (kHasZ) r.z = load_raw4_nb<T, kAligned>(z_row, t0 + 4 * q, L, pch_ok);
      else r.z = typename Raw4<T>::type{};
      r.C = elem_bits(Cp[c_row + min(t0 + c_step, L - 1)]);
    }
  };
  float dtsum = 0.0f;
  auto stage = [&](const Rows& r, int i, int sbuf) {
    const int t = tile_t(i) + 4 * q;
    float dv[4], yv[4], zv[4], de[4], dov[4];
    decode4(r.d, dv);
    decode4(r.y, yv);
    if constexpr (kHasZ) decode4(r.z, zv);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool valid = t + j >= vlo && t + j < vhi;
      const float x = dv[j] + Bias;
      const float dt = softplus ? softplus_t20(x) : x;
      de[j] = valid ? dt : 0.0f;
      const float dym = valid ? yv[j] : 0.0f;
      if constexpr (kHasZ) dov[j] = dym * (zv[j] * sigmoidf_fast(zv[j]));
      else dov[j] = dym;
      dtsum += de[j];
    }
    sSt[sbuf][0][q][row] = make_float4(de[0], de[1], de[2], de[3]);
    sSt[sbuf][1][q][row] = make_float4(dov[0], dov[1], dov[2], dov[3]);
    reinterpret_cast<float*>(&sC[sbuf][c_G][0])[2 * c_step + c_half] =
        c_ok ? bits_to_f32<T>(r.C) : 0.0f;
  };

  // Iteration i after barrier i stages tile i + 2 into buffer (i + 2) % 3
  // (last read during iteration i - 1); raw rows travel in a ring of kRing
  // tiles, loaded kRing iterations ahead of their staging.  Iterations run
  // in unrolled groups of four with no conditions around the memory
  // operations (work past the last tile is harmless: clamped loads, unread
  // buffers, masked sums).
  Rows rows[kRing];
#pragma unroll
  for (int k = 0; k < kRing; ++k) issue(rows[k], k);
  stage(rows[0], 0, 0);
  issue(rows[0], kRing);
  stage(rows[1 % kRing], 1, 1);
  issue(rows[1 % kRing], kRing + 1);
  __syncthreads();  // iteration 0
  stage(rows[2 % kRing], 2, 2);
  issue(rows[2 % kRing], kRing + 2);
  int sbuf = 0;  // staging buffer of tile i + 2
  for (int i0 = 1; i0 < nbar; i0 += 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = i0 + j;  // (i + 2) % kRing == (j + 3) % kRing (kRing divides 4)
      __syncthreads();
      stage(rows[(j + 3) % kRing], i + 2, sbuf);
      issue(rows[(j + 3) % kRing], i + 2 + kRing);
      sbuf = sbuf == kStage - 1 ? 0 : sbuf + 1;
    }
  }
  // the four lanes of a channel row are 4 consecutive lanes (q = lane % 4)
#pragma unroll
  for (int m = 1; m < kT4; m <<= 1) dtsum += __shfl_xor(dtsum, m, 64);
  if (q == 0 && pch_ok) seg_dt[sb * Dm + pch] = dtsum;
}

// Adds the partial sums: dB/dC over channel blocks, dA/dD/dbias over the
// (segment, batch row) rows, each in a fixed order.  kVec: dB/dC four
// consecutive elements per thread (128-bit partial loads, 4-element stores;
// batch * nstate * seqlen a multiple of 4 and dB/dC aligned), so a thread
// keeps nblk 16-byte loads in flight.
template <typename T, bool kVec>
__global__ __launch_bounds__(256) void scan_bwd_reduce_kernel(
    const int batch, const int rows, const int dim, const int N, const int L, const int nblk,
    const float* __restrict__ ws_bc, const float* __restrict__ ws_A,
    const float* __restrict__ ws_D, const float* __restrict__ ws_bias, T* __restrict__ dB,
    T* __restrict__ dC, float* __restrict__ dA, float* __restrict__ dD,
    float* __restrict__ dbias) {
  // the partial rows are bc_part_len(L) long; a work item sums 4 steps of one
  // (kind, b, n) row over the channel blocks, and writes the steps below L
  // (as one vector when kVec: L % 4 == 0 and dB / dC 4-element aligned)
  const int Lp = bc_part_len(L), L4 = Lp / 4;
  const size_t nrow = (size_t)batch * N;
  const size_t nBC = nrow * Lp;
  const size_t nA = (size_t)dim * N;
  const size_t nbc_items = 2 * nrow * L4;
  const size_t total = nbc_items + nA + dim;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    if (i < nbc_items) {
      const size_t rr = i / L4;  // kind * nrow + row
      const int t = (int)(i % L4) * 4;
      const size_t kind = rr / nrow, r = rr % nrow;
      const float* src = ws_bc + kind * nblk * nBC + r * Lp + t;
      auto part = [&](int k) { return *reinterpret_cast<const float4*>(src + (size_t)k * nBC); };
      auto add = [](float4& a, const float4& v) { a.x += v.x; a.y += v.y; a.z += v.z; a.w += v.w; };
      // 4 partial loads in flight per thread (8, 16 and 32 were slower), into
      // four accumulators (blocks k = 4m + j into a_j, the remainder into a_0)
      // added pairwise at the end: a term passes through about nblk / 4 + 2
      // additions instead of nblk, in a fixed order
      const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
      float4 a0 = zero, a1 = zero, a2 = zero, a3 = zero;
      int k = 0;
      for (; k + 4 <= nblk; k += 4) {
        const float4 v0 = part(k), v1 = part(k + 1), v2 = part(k + 2), v3 = part(k + 3);
        add(a0, v0); add(a1, v1); add(a2, v2); add(a3, v3);
      }
      for (; k < nblk; ++k) add(a0, part(k));
      add(a0, a1);
      add(a2, a3);
      float4 s4 = a0;
      add(s4, a2);
      const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
      T* dst = (kind ? dC : dB) + r * L + t;
      if (kVec && t + 4 <= L) {
        if constexpr (sizeof(T) == 4) {
          *reinterpret_cast<float4*>(dst) = s4;
        } else {
          *reinterpret_cast<uint2*>(dst) =
              make_uint2(pack_bf16x2(sv[0], sv[1]), pack_bf16x2(sv[2], sv[3]));
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (t + j < L) Elem<T>::store1(dst + j, sv[j]);
      }
    } else if (i < nbc_items + nA) {
      const size_t r = i - nbc_items;
      float acc = 0.0f;
      for (int bb = 0; bb < rows; ++bb) acc += ws_A[(size_t)bb * nA + r];
      dA[r] = acc;
    } else {
      const size_t d = i - nbc_items - nA;
      float sd = 0.0f, sb = 0.0f;
      for (int bb = 0; bb < rows; ++bb) {
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

template <typename T, int kSG, bool kHasZ, bool kAligned, bool kPart>
static hipError_t launch_bwd4(const ScanParams& p, const float* bc, hipStream_t st) {
  const int nsc = kPart ? p.nsc : 1;
  // the role-split kernels' buffer ranges must fit 2^31 bytes: a wave's 16
  // channel rows, all of the dB/dC partials, and a batch row's saved states
  const bool ws =
      kSG == 1 && !kPart && (size_t)(kBlockCh / kWsProd) * p.seqlen * sizeof(T) < (1u << 31) &&
      2 * (size_t)p.nblk * p.batch * p.nstate * bc_part_len(p.seqlen) * sizeof(float) < (1u << 31) &&
      (size_t)p.nchunks * p.nstate * p.hs * p.dim * sizeof(float) < (1u << 31);
  if (p.nseg > 1) {
    ProfScope prof("scan_bwd_segsum", st);
    // the role-split summaries per sub-segment (p.sub_k per segment), the
    // general ones per segment
    if (ws) {
      hipLaunchKernelGGL((scan_bwd_segsum_ws_kernel<T, kHasZ, kAligned>),
                         dim3(p.nblk, p.batch, (p.nseg - 1) * p.sub_k), dim3(kWsThreads), 0, st,
                         dims_of(p), (const T*)p.delta, (const T*)p.dout, (const T*)p.z, p.A,
                         (const T*)p.C, p.bias, p.length, p.seg_h, p.seg_dt);
    } else {
      // only these summaries read the prepped B/C layout
      hipError_t e = launch_bc_prep(p, sizeof(T) == 2 ? 1 : 0, const_cast<float*>(bc), st);
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL((scan_bwd_segsum_kernel<T, kSG, kHasZ, kAligned>),
                         dim3(p.nblk, p.batch, (p.nseg - 1) * nsc), dim3(kThreads), 0, st,
                         dims_of(p), (const T*)p.delta, (const T*)p.dout, (const T*)p.z, p.A, bc,
                         p.bias, p.length, p.seg_h, p.seg_dt);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  dim3 grid(p.nblk, p.batch, p.nseg * nsc);
  if (ws) {
    ProfScope prof("scan_bwd", st);
    hipLaunchKernelGGL((scan_bwd_ws_kernel<T, kHasZ, kAligned>), grid, dim3(kWsThreads), 0, st,
                       dims_of(p), (const T*)p.u, (const T*)p.delta, p.A, (const T*)p.B,
                       (const T*)p.C, p.D, p.bias, p.h_init, p.length, (const T*)p.z,
                       (const T*)p.out_ungated, p.h_chunks_in, (const T*)p.dout, p.dh_last,
                       (T*)p.du, (T*)p.ddelta, (T*)p.dz, p.dh_init, p.ws_bc, p.ws_A, p.ws_D,
                       p.ws_bias, p.dummy, p.seg_h, p.seg_dt);
    return hipGetLastError();
  }
  {
    ProfScope prof("scan_bwd", st);
    hipLaunchKernelGGL((scan_bwd_kernel<T, kSG, kHasZ, kAligned, kPart>), grid, dim3(kThreads), 0,
                       st, dims_of(p), (const T*)p.u, (const T*)p.delta, p.A, (const T*)p.B,
                       (const T*)p.C, p.D, p.bias, p.h_init, p.length, (const T*)p.z,
                       (const T*)p.out_ungated, p.h_chunks_in, (const T*)p.dout, p.dh_last,
                       (T*)p.du, (T*)p.ddelta, (T*)p.dz, p.dh_init, p.ws_bc, p.ws_A, p.ws_D,
                       p.ws_bias, p.dummy, p.seg_h, p.seg_dt, p.ws_gb, p.ws_gd);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if constexpr (kPart) {
    ProfScope prof("scan_bwd_combine", st);
    hipLaunchKernelGGL((scan_bwd_combine_kernel<T, kHasZ>), dim3(p.dim, p.batch), dim3(256), 0,
                       st, dims_of(p), p.nsc, (const T*)p.u, (const T*)p.delta, (const T*)p.dout,
                       (const T*)p.z, p.D, p.bias, p.length, p.ws_gb, p.ws_gd, (T*)p.du,
                       (T*)p.ddelta, p.ws_D, p.ws_bias);
  }
  return hipGetLastError();
}

template <typename T, int kSG, bool kPart = false>
static hipError_t launch_bwd3(const ScanParams& p, const float* bc, bool aligned, hipStream_t st) {
  if (p.z)
    return aligned ? launch_bwd4<T, kSG, true, true, kPart>(p, bc, st)
                   : launch_bwd4<T, kSG, true, false, kPart>(p, bc, st);
  return aligned ? launch_bwd4<T, kSG, false, true, kPart>(p, bc, st)
                 : launch_bwd4<T, kSG, false, false, kPart>(p, bc, st);
}

template <typename T>
static hipError_t launch_bwd2(const ScanParams& p, const float* bc, bool aligned, hipStream_t st) {
  hipError_t e;
  if (p.nstate <= 16) e = launch_bwd3<T, 1>(p, bc, aligned, st);
  else if (p.nstate <= 32) e = launch_bwd3<T, 2>(p, bc, aligned, st);
  else if (p.nstate <= kBwdChunkStates) e = launch_bwd3<T, 4>(p, bc, aligned, st);
  else e = launch_bwd3<T, 4, true>(p, bc, aligned, st);
  if (e != hipSuccess) return e;
  const uintptr_t vec_align = 4 * sizeof(T);
  const bool vec = p.seqlen % 4 == 0 && (uintptr_t)p.dB % vec_align == 0 &&
                   (uintptr_t)p.dC % vec_align == 0;
  const size_t total = 2 * (size_t)p.batch * p.nstate * (bc_part_len(p.seqlen) / 4) +
                       (size_t)p.dim * p.nstate + p.dim;
  const int blocks = (int)std::min<size_t>((total + 255) / 256, 16384);
  ProfScope prof("scan_bwd_reduce", st);
  if (vec)
    hipLaunchKernelGGL((scan_bwd_reduce_kernel<T, true>), dim3(blocks), dim3(256), 0, st, p.batch,
                       p.batch * p.nseg, p.dim, p.nstate, p.seqlen, p.nblk, p.ws_bc, p.ws_A,
                       p.ws_D, p.ws_bias, (T*)p.dB, (T*)p.dC, p.dA, p.dD, p.dbias);
  else
    hipLaunchKernelGGL((scan_bwd_reduce_kernel<T, false>), dim3(blocks), dim3(256), 0, st, p.batch,
                       p.batch * p.nseg, p.dim, p.nstate, p.seqlen, p.nblk, p.ws_bc, p.ws_A,
                       p.ws_D, p.ws_bias, (T*)p.dB, (T*)p.dC, p.dA, p.dD, p.dbias);
  return hipGetLastError();
}

// bc must hold bc_prep_floats() floats; ws_* are laid out by the caller.
// nstate <= 256 (past 64: p.nsc chunks with p.ws_gb / p.ws_gd).
hipError_t launch_scan_bwd(const ScanParams& p, int dtype, bool aligned, float* bc,
                           hipStream_t st) {
  if (dtype == 1) return launch_bwd2<__hip_bfloat16>(p, bc, aligned, st);
  return launch_bwd2<float>(p, bc, aligned, st);
}

}  // namespace ssm
