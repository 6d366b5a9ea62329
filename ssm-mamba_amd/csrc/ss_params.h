// Kernel argument blocks for the selective-scan and state-update kernels.
// All tensors are dense and row-major:
//   u, delta, z, out, dout, du, ddelta, dz : (batch, dim, seqlen)
//   B, C, dB, dC                           : (batch, nstate, seqlen)
//   A, dA                                  : (dim, nstate)          fp32
//   D, delta_bias, dD, ddelta_bias         : (dim,)                 fp32
//   h_init, h_last, dh_last, dh_init       : (batch, dim, nstate)   fp32
//   h_chunks                               : (batch, nchunks, nstate, dim) fp32,
//                                            state after each kChunk steps
//                                            (nchunks: the slots of a batch row,
//                                            ceil(seqlen / kChunk), or 8 per
//                                            128-step chunk in the pair layout)
//   length                                 : (batch,) int64
#pragma once

#include <stdint.h>

namespace ssm {

constexpr int kChunk = 16;    // steps between saved states
constexpr int kTileF = 32;    // steps staged through LDS per forward tile
constexpr int kSubF = 4;      // forward sub-tiles staged (and loaded) together
constexpr int kTileB = 16;    // steps staged through LDS per backward tile
constexpr int kBlockCh = 64;  // channels per workgroup (one per lane)
constexpr int kWaves = 8;     // waves per workgroup; wave w owns state pairs G = g*8 + w
constexpr int kThreads = 64 * kWaves;
// role-split kernels (N <= 16): consumer waves run the recurrences, producer
// waves stage tiles and finish per-position outputs
constexpr int kWsCons = 8;    // consumer waves: state pair w
constexpr int kWsProd = 4;    // producer waves: (channel row, 4-step column) per lane
constexpr int kWsThreads = 64 * (kWsCons + kWsProd);

// Scalar shape/flag block passed to the scan kernels (pointers travel as
// separate __restrict__ kernel arguments).
struct ScanDims {
  int batch, dim, seqlen, nstate, nchunks, nblk;
  int pad_right;
  int softplus;
  int seg_len;  // steps per sequence segment (a multiple of the forward super-tile)
  int nseg;     // segments (1: the whole row in one workgroup)
  int sub_k;    // summaries per segment (sub-segments of sub_span(seg_len, sub_k) steps)
  int64_t bc_bstride;  // elements between batch rows of B and of C (rows of a batch are seqlen apart)
  int hs;              // h_chunks state-slot stride in rows of dim (1: states only; 2: (prod a, h) pairs)
};

// The step-size projection of a Mamba block fused into the role-split
// forward (modules/mamba.py:141-160): the block's x-projection output
// ssm_params is token-major, (batch, seqlen, P) with P = rank + 2 N and each
// token's row [dt (rank) | B (N) | C (N)], and the scan's step sizes are
// delta_raw = W_dt dt rounded to bf16 (the reference's delta matrix product
// in the model dtype), with W_dt (dim, rank).  Each producer wave computes
// its 16 channels x 16 steps of delta_raw per tile with kDtK
// v_mfma_f32_16x16x32_bf16 (32 ranks each) and reads B and C in place from
// the same rows, so neither delta nor channel-major copies of B and C are
// written or read.  Operand layout of the 16x16x32 bf16 MFMA (checked on
// gfx950): lane l supplies A[l % 16][8 (l / 16) + i] and B[8 (l / 16) + i][l % 16],
// i = 0..7, and holds D[4 (l / 16) + r][l % 16] in accumulator r.  Here A is
// dt^T (16 steps x 32 ranks: one 16-byte load from a token row per lane and
// k-step), B is W_dt^T (32 ranks x 16 channels: 16 bytes of a W_dt row, held
// for the whole launch), and D is delta_raw (steps x channels).
struct DtProj {
  const void* params;   // (batch, seqlen, P) bf16, 16-byte aligned rows
  int64_t pstride;      // elements between batch rows of params
  int P, rank;
  const void* w;        // (dim, rank) bf16
  void* delta_out;      // nullable: delta_raw as (batch, dim, seqlen) bf16
  int64_t zbstride;     // elements between batch rows of z (>= dim * seqlen)
};
constexpr int kDtK = 2;  // MFMA k-steps of 32 ranks: rank <= 64

// Sub-segments of the segment summaries: segment s is cut into sub_k parts
// of sub_span steps (a multiple of the 32-step summary tile), the last part
// ending at the segment's end (shorter, or empty when the others already
// cover the segment).
#if defined(__HIPCC__)
__host__ __device__
#endif
inline int sub_span(int seg_len, int sub_k) {
  return ((seg_len + sub_k - 1) / sub_k + kTileF - 1) / kTileF * kTileF;
}

// Steps [t0, t1) of summary z = s * sub_k + j (part j of segment s); t1 <= t0
// for an empty part.
#if defined(__HIPCC__)
__host__ __device__
#endif
inline void sub_range(const ScanDims& p, int z, int& t0, int& t1) {
  const int s = z / p.sub_k, j = z % p.sub_k;
  const int span = sub_span(p.seg_len, p.sub_k);
  const int base = s * p.seg_len;
  t0 = base + (j * span < p.seg_len ? j * span : p.seg_len);
  const int e = base + ((j + 1) * span < p.seg_len ? (j + 1) * span : p.seg_len);
  t1 = e < p.seqlen ? e : p.seqlen;
}

struct ScanParams {
  int batch, dim, seqlen, nstate, nchunks, nblk;
  int pad_right;  // 1: valid t < len; 0: valid t >= seqlen - len
  int softplus;   // 1: delta = softplus(delta + bias); 0: delta + bias

  const void* u;
  const void* delta;
  const float* A;
  const void* B;
  const void* C;
  int64_t bc_bstride;  // elements between batch rows of B and of C
  const float* D;      // nullable
  const float* bias;   // nullable
  const float* h_init; // nullable
  const int64_t* length;  // nullable
  const void* z;       // nullable
  // ungated output D*u + sum_n C*h (with z): written by the forward when
  // non-null, read by the backward for dz
  void* out_ungated;

  // forward outputs
  void* out;
  // nullable (then h_last).  Row (b, chunk c, state n) of dim floats starts at
  // h_chunks + ((b * nchunks + c) * nstate * hs + n * hs) * dim: hs = 1 is the
  // (batch, nchunks, nstate, dim) state layout; hs = 2 interleaves a second
  // row per state (the caller offsets h_chunks by one row to write the odd
  // slots of a (batch, nchunks, 2 * nstate, dim) pair layout)
  float* h_chunks;
  int hs;
  float* h_last;    // nullable

  // backward
  const float* h_chunks_in;
  const void* dout;
  const float* dh_last;  // nullable
  void* du;
  void* ddelta;
  void* dz;          // nullable (needs z)
  float* dh_init;    // nullable (needs h_init)
  float* ws_bc;      // (2, nblk, batch, nstate, seqlen) dB/dC partial sums per channel block
  float* ws_A;       // (batch, dim, nstate) dA partial sums per batch row
  float* ws_D;       // (batch, dim)
  float* ws_bias;    // (batch, dim)
  float* dA;
  void* dB;
  void* dC;
  float* dD;      // nullable
  float* dbias;   // nullable

  // 256 bytes of workspace that masked-off lanes store to (never read), so
  // the kernels' steady-state stores need no branches
  void* dummy;

  // sequence split (nseg > 1).  Forward: per sub-segment j (seg_len / sub_k
  // steps) of segments 0 .. nseg - 2, the state its steps produce from zero,
  // ((nseg - 1) * sub_k, batch, nstate, dim), and the sum of its step sizes,
  // ((nseg - 1) * sub_k, batch, dim).  Backward (sub_k = 1): the per-segment
  // adjoint carries and step sums of segments 1 .. nseg - 1.
  int seg_len, nseg, sub_k;
  float* seg_h;
  float* seg_dt;

  // backward past 64 states: nsc chunks of 64 states, each leaving its
  // per-position sums over its states, (nsc, batch, dim, seqlen) fp32
  int nsc;
  float* ws_gb;  // sum_n G B
  float* ws_gd;  // sum_n A G a h_{t-1}
};

// states per backward workgroup (8 waves x 4 pairs); larger counts run in
// chunks of this many
constexpr int kBwdChunkStates = 64;

constexpr size_t kDummyBytes = 256;

struct UpdateParams {
  int batch, dim, nstate, softplus;
  const float* state;
  float* new_state;  // may alias state
  const void* x;
  const void* dt;
  const float* A;
  const void* B;
  const void* C;
  const float* D;      // nullable
  const float* bias;   // nullable
  const void* z;       // nullable
  void* out;
};

inline ScanDims dims_of(const ScanParams& p) {
  return ScanDims{p.batch,    p.dim,     p.seqlen,  p.nstate, p.nchunks, p.nblk,
                  p.pad_right, p.softplus, p.seg_len, p.nseg,   p.sub_k,  p.bc_bstride,
                  p.hs > 1 ? p.hs : 1};
}

}  // namespace ssm
