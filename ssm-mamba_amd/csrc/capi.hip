// C ABI of the selective-scan library: argument validation, workspace
// carving, dispatch to the gfx950 kernels.  See include/ssm_mamba.h.
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/ssm_mamba.h"
#include "ss_io.cuh"
#include "ss_params.h"
#include "ss_prof.h"
#include <mutex>
#include <vector>

namespace ssm {
hipError_t launch_scan_fwd(const ScanParams& p, int dtype, bool aligned, float* bc, hipStream_t st);
hipError_t launch_scan_bwd(const ScanParams& p, int dtype, bool aligned, float* bc, hipStream_t st);
hipError_t launch_chunk_decay(const ScanParams& p, int dtype, float* pairs, hipStream_t st);
hipError_t launch_chunk_tail(const ScanParams& p, float* pairs, hipStream_t st);
bool scan_fwd_dt_supported(const ScanParams& p);
hipError_t launch_scan_fwd_dt(const ScanParams& p, const DtProj& dt, bool aligned, hipStream_t st);
hipError_t launch_state_update(const UpdateParams& p, int dtype, bool vecN, hipStream_t st);
size_t bc_prep_floats(int batch, int nstate, int seqlen);
size_t bwd_ws_floats(int batch, int dim, int nstate, int seqlen);
void fwd_segments(int batch, int nblk, int seqlen, int& nseg, int& seg_len);
size_t fwd_seg_floats(int batch, int dim, int nstate, int seqlen);
int fwd_summary_split(int batch, int nblk, int nseg, int seg_len);
int conv1d_max_width();
int decode_max_batch();
int decode_xproj_blocks(int64_t dim, int64_t nout);
hipError_t launch_decode_gemv(int bf16, const void* W, const void* x, const void* nw, float eps,
                              const void* bias, const void* res, void* y, int B, int O, int K,
                              hipStream_t st);
hipError_t launch_decode_in_proj_conv(int bf16, const void* W, const void* x, const void* nw,
                                      float eps, const void* bias, void* xz, int B, int dim, int K,
                                      int width, void* ctx, const void* cw, const void* cb,
                                      void* xc, const void* Wx, int nout, float* part,
                                      hipStream_t st);
hipError_t launch_decode_ssm_step(int bf16, const void* p, int nout, int nparts, int R,
                                  const void* Wdt, const void* dtb, const void* logA, const void* D,
                                  const void* xc, const void* xz, int ld, float* state, void* y,
                                  int B, int dim, int nstate, bool vecR, hipStream_t st);
int64_t decode_layers_workspace(int B, int nlayers, int K, int dim, int nout, int bf16);
const char* decode_layers_unsupported(int K, int dim, int nout, int bf16);
int64_t decode_layers_error_offset();
int64_t decode_pick_workspace(int B);
hipError_t launch_decode_pick(int bf16, const void* p, int B, int V, int64_t* token,
                              int64_t* tokens, int64_t ld, int64_t cols, int64_t* pos, void* ws,
                              hipStream_t st);
int decode_layers_grid(int B, int K, int dim);
int decode_layers_max_width();
hipError_t launch_decode_layers(int bf16, const void* table, int nlayers, int B, int K, int dim,
                                int width, int R, int nout, float eps, const void* x, void* out,
                                void* ws, hipStream_t st);
hipError_t launch_rms_norm_cm(int bf16, const void* x, const void* w, float eps, void* out, int B,
                              int C, int L, bool pair, hipStream_t st);
hipError_t launch_causal_conv1d_fwd(int batch, int dim, int L, int K, int dtype_bf16,
                                    const void* x, int64_t xbs, const void* w, const void* bias,
                                    int silu, void* out, const int64_t* lengths, void* window,
                                    bool vec, hipStream_t st);
hipError_t launch_causal_conv1d_bwd(int batch, int dim, int L, int K, int dtype_bf16,
                                    const void* x, const void* w, const void* bias,
                                    const void* dout, int silu, void* dx, void* dw, void* dbias,
                                    float* part, bool vec, hipStream_t st);
}  // namespace ssm

namespace ssm {

// ---- kernel timing (see ss_prof.h)
namespace {
struct ProfRec {
  const char* name;
  hipEvent_t a, b;
};
std::mutex g_prof_mu;
bool g_prof_on = false;
std::vector<hipEvent_t> g_prof_pool;
std::vector<ProfRec> g_prof_recs;
constexpr size_t kProfPool = 8192;
}  // namespace

ProfScope::ProfScope(const char* name, hipStream_t st) : slot_(-1), st_(st) {
  if (!g_prof_on) return;
  std::lock_guard<std::mutex> lk(g_prof_mu);
  const size_t used = g_prof_recs.size() * 2;
  if (!g_prof_on || used + 2 > g_prof_pool.size()) return;
  ProfRec r{name, g_prof_pool[used], g_prof_pool[used + 1]};
  if (hipEventRecord(r.a, st) != hipSuccess) return;
  slot_ = (int)g_prof_recs.size();
  g_prof_recs.push_back(r);
}

ProfScope::~ProfScope() {
  if (slot_ < 0) return;
  std::lock_guard<std::mutex> lk(g_prof_mu);
  (void)hipEventRecord(g_prof_recs[slot_].b, st_);
}

}  // namespace ssm

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return SSM_OK;
  return fail(SSM_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned16(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

size_t round256(size_t bytes) { return (bytes + 255) & ~(size_t)255; }

// state chunks of the backward past ssm::kBwdChunkStates states (0: one pass)
// Row length of the backward's dB/dC partials: seqlen padded to whole 16-step
// tiles (bc_part_len in scan_bwd.hip).
size_t bwd_part_len(int64_t seqlen) { return (size_t)(seqlen + ssm::kTileB - 1) / ssm::kTileB * ssm::kTileB; }

size_t bwd_chunks(int64_t nstate) {
  return nstate > ssm::kBwdChunkStates
             ? (size_t)((nstate + ssm::kBwdChunkStates - 1) / ssm::kBwdChunkStates)
             : 0;
}

int check_common(int64_t batch, int64_t dim, int64_t seqlen, int64_t nstate, int dtype,
                 int max_nstate) {
  if (dtype != SSM_F32 && dtype != SSM_BF16)
    return fail(SSM_ERR_INVALID, "dtype must be SSM_F32 or SSM_BF16 (got %d)", dtype);
  if (batch < 1 || dim < 1 || seqlen < 1 || nstate < 1)
    return fail(SSM_ERR_INVALID, "batch, dim, seqlen and nstate must be >= 1 (got %lld, %lld, %lld, %lld)",
                (long long)batch, (long long)dim, (long long)seqlen, (long long)nstate);
  if (nstate > max_nstate)
    return fail(SSM_ERR_UNSUPPORTED, "selective_scan only supports state_dim <= %d (got %lld)",
                max_nstate, (long long)nstate);
  if (batch > 65535) return fail(SSM_ERR_UNSUPPORTED, "batch must be <= 65535 (got %lld)", (long long)batch);
  if (dim > INT_MAX / 2 || seqlen > INT_MAX / 2)
    return fail(SSM_ERR_UNSUPPORTED, "dim and seqlen must be < 2^30");
  return SSM_OK;
}

ssm::ScanParams make_scan_params(int64_t batch, int64_t dim, int64_t seqlen, int64_t nstate,
                                 const void* u, const void* delta, const float* A, const void* B,
                                 const void* C, int64_t bc_batch_stride, const float* D,
                                 const float* delta_bias,
                                 const float* h_init, const int64_t* length, int padding_right,
                                 const void* z, int delta_softplus) {
  ssm::ScanParams p{};
  p.batch = (int)batch;
  p.dim = (int)dim;
  p.seqlen = (int)seqlen;
  p.nstate = (int)nstate;
  p.nchunks = (int)((seqlen + ssm::kChunk - 1) / ssm::kChunk);
  p.nblk = (int)((dim + ssm::kBlockCh - 1) / ssm::kBlockCh);
  p.pad_right = padding_right ? 1 : 0;
  p.softplus = delta_softplus ? 1 : 0;
  p.u = u;
  p.delta = delta;
  p.A = A;
  p.B = B;
  p.C = C;
  p.bc_bstride = bc_batch_stride ? bc_batch_stride : nstate * seqlen;
  p.D = D;
  p.bias = delta_bias;
  p.h_init = h_init;
  p.length = length;
  p.z = z;
  p.seg_len = (int)seqlen;
  p.nseg = 1;
  p.sub_k = 1;
  return p;
}

int check_conv(int64_t batch, int64_t dim, int64_t seqlen, int64_t width, int dtype) {
  if (dtype != SSM_F32 && dtype != SSM_BF16)
    return fail(SSM_ERR_INVALID, "dtype must be SSM_F32 or SSM_BF16 (got %d)", dtype);
  if (batch < 1 || dim < 1 || seqlen < 1 || width < 1)
    return fail(SSM_ERR_INVALID, "batch, dim, seqlen and width must be >= 1 (got %lld, %lld, %lld, %lld)",
                (long long)batch, (long long)dim, (long long)seqlen, (long long)width);
  if (width > ssm::conv1d_max_width())
    return fail(SSM_ERR_UNSUPPORTED, "causal_conv1d supports width <= %d (got %lld)",
                ssm::conv1d_max_width(), (long long)width);
  if (batch * dim > INT_MAX || seqlen > INT_MAX / 2)
    return fail(SSM_ERR_UNSUPPORTED, "batch * dim must be < 2^31 and seqlen < 2^30");
  return SSM_OK;
}

int check_decode(int64_t batch, int dtype) {
  if (dtype != SSM_F32 && dtype != SSM_BF16)
    return fail(SSM_ERR_INVALID, "dtype must be SSM_F32 or SSM_BF16 (got %d)", dtype);
  if (batch < 1 || batch > ssm::decode_max_batch())
    return fail(SSM_ERR_UNSUPPORTED, "decode kernels take 1 <= batch <= %d (got %lld)",
                ssm::decode_max_batch(), (long long)batch);
  return SSM_OK;
}

// elements of the streamed type per 16-byte access
int elems16(int dtype) { return dtype == SSM_BF16 ? 8 : 4; }

bool scan_aligned(int dtype, int64_t seqlen, std::initializer_list<const void*> ptrs) {
  const int vec = dtype == SSM_BF16 ? 8 : 4;
  if (seqlen % vec) return false;
  for (const void* p : ptrs)
    if (!aligned16(p)) return false;
  return true;
}

}  // namespace

// ---- static scratch of the allocation-free forward
//
// Device memory for ssm_selective_scan_fwd_noalloc's workspace (prepped B/C,
// sequence-split summaries, store sink): every GPU the library runs on holds
// its own copy for the life of the process.  Host code never uses the
// array's name as an address: each device's copy is found once with
// hipGetSymbolAddress (with that device current) and kept in g_scratch.
static __device__ __align__(256) unsigned char scratch[SSM_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

// The device address of the current device's scratch copy.
int scratch_on_current_device(void** out) {
  int dev = -1;
  if (int e = hip_status(hipGetDevice(&dev), "hipGetDevice")) return e;
  if (dev < 0 || dev >= kMaxDevices)
    return fail(SSM_ERR_UNSUPPORTED, "device index %d out of range (< %d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    if (int e = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                           "hipGetSymbolAddress(scratch)"))
      return e;
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return SSM_OK;
}
}  // namespace

extern "C" {

const char* ssm_last_error(void) { return g_err.c_str(); }

int ssm_abi_version(void) { return 10; }

int ssm_profile_begin(void) {
  g_err.clear();
  std::lock_guard<std::mutex> lk(ssm::g_prof_mu);
  while (ssm::g_prof_pool.size() < ssm::kProfPool) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return fail(SSM_ERR_HIP, "hipEventCreate failed");
    ssm::g_prof_pool.push_back(e);
  }
  ssm::g_prof_recs.clear();
  ssm::g_prof_on = true;
  return SSM_OK;
}

int ssm_profile_end(char* buf, size_t buf_bytes) {
  g_err.clear();
  std::lock_guard<std::mutex> lk(ssm::g_prof_mu);
  ssm::g_prof_on = false;
  std::vector<std::pair<std::string, std::pair<int, double>>> agg;
  for (const auto& r : ssm::g_prof_recs) {
    if (hipEventSynchronize(r.b) != hipSuccess) return fail(SSM_ERR_HIP, "hipEventSynchronize failed");
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess)
      return fail(SSM_ERR_HIP, "hipEventElapsedTime failed");
    bool found = false;
    for (auto& e : agg)
      if (e.first == r.name) {
        e.second.first += 1;
        e.second.second += ms;
        found = true;
      }
    if (!found) agg.push_back({r.name, {1, (double)ms}});
  }
  std::string out;
  for (const auto& e : agg) {
    char line[160];
    snprintf(line, sizeof(line), "%s %d %.6f\n", e.first.c_str(), e.second.first, e.second.second);
    out += line;
  }
  if (buf && buf_bytes) {
    const size_t n = std::min(out.size(), buf_bytes - 1);
    memcpy(buf, out.data(), n);
    buf[n] = 0;
  }
  const int nrec = (int)ssm::g_prof_recs.size();
  ssm::g_prof_recs.clear();
  return nrec;
}

int64_t ssm_scan_nchunks(int64_t seqlen) { return seqlen <= 0 ? 0 : (seqlen + SSM_CHUNK - 1) / SSM_CHUNK; }
int64_t ssm_scan_ref_nchunks(int64_t seqlen) {
  return seqlen <= 0 ? 0 : (seqlen + SSM_REF_CHUNK - 1) / SSM_REF_CHUNK;
}

size_t ssm_scan_fwd_workspace_bytes(int64_t batch, int64_t dim, int64_t seqlen, int64_t nstate) {
  if (batch < 1 || dim < 1 || seqlen < 1 || nstate < 1) return 0;
  return round256(ssm::bc_prep_floats((int)batch, (int)nstate, (int)seqlen) * sizeof(float)) +
         round256(ssm::fwd_seg_floats((int)batch, (int)dim, (int)nstate, (int)seqlen) *
                  sizeof(float)) +
         ssm::kDummyBytes;
}

size_t ssm_scan_bwd_workspace_bytes(int64_t batch, int64_t dim, int64_t seqlen, int64_t nstate) {
  if (batch < 1 || dim < 1 || seqlen < 1 || nstate < 1) return 0;
  const size_t nblk = (dim + ssm::kBlockCh - 1) / ssm::kBlockCh;
  int nseg, seg_len;
  ssm::fwd_segments((int)batch, (int)nblk, (int)seqlen, nseg, seg_len);
  const size_t rows = (size_t)batch * nseg;  // (segment, batch row) partial rows
  return round256(ssm::bc_prep_floats((int)batch, (int)nstate, (int)seqlen) * sizeof(float)) +
         round256(2 * nblk * batch * nstate * bwd_part_len(seqlen) * sizeof(float)) +
         round256(rows * dim * nstate * sizeof(float)) +
         2 * round256(rows * dim * sizeof(float)) +
         round256(ssm::fwd_seg_floats((int)batch, (int)dim, (int)nstate, (int)seqlen) *
                  sizeof(float)) +
         2 * round256(bwd_chunks(nstate) * batch * dim * seqlen * sizeof(float)) +
         ssm::kDummyBytes;
}

int ssm_selective_scan_fwd(int64_t batch, int64_t dim, int64_t seqlen, int64_t nstate, int dtype,
                           const void* u, const void* delta, const float* A, const void* B,
                           const void* C, int64_t bc_batch_stride, const float* D,
                           const float* delta_bias,
                           const float* h_init, const int64_t* length, int padding_right,
                           const void* z, int delta_softplus, void* out, void* out_ungated,
                           float* h_chunks, int h_pairs, float* h_last, void* workspace,
                           size_t workspace_bytes, void* stream) {
  g_err.clear();
  if (int e = check_common(batch, dim, seqlen, nstate, dtype, 256)) return e;
  if (!u || !delta || !A || !B || !C || !out)
    return fail(SSM_ERR_INVALID, "u, delta, A, B, C and out must be non-NULL");
  if (out_ungated && !z) return fail(SSM_ERR_INVALID, "out_ungated requires z");
  if (h_pairs && !h_chunks) return fail(SSM_ERR_INVALID, "h_pairs requires h_chunks");
  const size_t need = ssm_scan_fwd_workspace_bytes(batch, dim, seqlen, nstate);
  if (!workspace || workspace_bytes < need)
    return fail(SSM_ERR_INVALID, "workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
  if (bc_batch_stride != 0 && bc_batch_stride < nstate * seqlen)
    return fail(SSM_ERR_INVALID, "bc_batch_stride must be 0 (contiguous) or at least nstate * seqlen (got %lld)",
                (long long)bc_batch_stride);
  ssm::ScanParams p = make_scan_params(batch, dim, seqlen, nstate, u, delta, A, B, C,
                                       bc_batch_stride, D, delta_bias,
                                       h_init, length, padding_right, z, delta_softplus);
  p.out = out;
  p.out_ungated = out_ungated;
  // pair layout: the states go to the odd rows (one row of dim in), the
  // chunk decays to the even rows of each 128-step chunk's carry slot; a
  // batch row holds SSM_REF_SLOTS slots per 128-step chunk
  p.h_chunks = (h_chunks && h_pairs) ? h_chunks + dim : h_chunks;
  p.hs = h_pairs ? 2 : 1;
  if (h_pairs) p.nchunks = (int)(SSM_REF_SLOTS * ssm_scan_ref_nchunks(seqlen));
  p.h_last = h_last;
  // workspace: [prepped B/C][segment states and step sums][dummy]
  char* ws = static_cast<char*>(workspace) +
             round256(ssm::bc_prep_floats((int)batch, (int)nstate, (int)seqlen) * sizeof(float));
  ssm::fwd_segments((int)batch, p.nblk, (int)seqlen, p.nseg, p.seg_len);
  p.sub_k = ssm::fwd_summary_split((int)batch, p.nblk, p.nseg, p.seg_len);
  p.seg_h = reinterpret_cast<float*>(ws);
  p.seg_dt = p.seg_h + (size_t)(p.nseg - 1) * p.sub_k * batch * nstate * dim;
  ws += round256(ssm::fwd_seg_floats((int)batch, (int)dim, (int)nstate, (int)seqlen) * sizeof(float));
  p.dummy = ws;
  const bool aligned = scan_aligned(dtype, seqlen, {u, delta, z, out, out_ungated});
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (h_pairs) {
    if (int e = hip_status(ssm::launch_chunk_decay(p, dtype, h_chunks, st),
                           "selective_scan chunk decay launch"))
      return e;
  }
  if (int e = hip_status(ssm::launch_scan_fwd(p, dtype, aligned, static_cast<float*>(workspace), st),
                         "selective_scan forward launch"))
    return e;
  if (h_pairs)
    return hip_status(ssm::launch_chunk_tail(p, h_chunks, st), "selective_scan chunk tail launch");
  return SSM_OK;
}

int ssm_selective_scan_bwd(int64_t batch, int64_t dim, int64_t seqlen, int64_t nstate, int dtype,
                           const void* u, const void* delta, const float* A, const void* B,
                           const void* C, int64_t bc_batch_stride, const float* D,
                           const float* delta_bias,
                           const float* h_init, const int64_t* length, int padding_right,
                           const void* z, const void* out_ungated, int delta_softplus,
                           const float* h_chunks, int h_pairs, const void* dout,
                           const float* dh_last, void* du, void* ddelta,
                           float* dA, void* dB, void* dC, float* dD, float* ddelta_bias,
                           float* dh_init, void* dz, void* workspace, size_t workspace_bytes,
                           void* stream) {
  g_err.clear();
  if (int e = check_common(batch, dim, seqlen, nstate, dtype, 256)) return e;
  if (!u || !delta || !A || !B || !C || !h_chunks || !dout || !du || !ddelta || !dA || !dB || !dC)
    return fail(SSM_ERR_INVALID,
                "u, delta, A, B, C, h_chunks, dout, du, ddelta, dA, dB and dC must be non-NULL");
  if (dh_init && !h_init) return fail(SSM_ERR_INVALID, "dh_init requires h_init");
  if ((dz || out_ungated) && !z) return fail(SSM_ERR_INVALID, "dz and out_ungated require z");
  if (z && (!dz || !out_ungated))
    return fail(SSM_ERR_INVALID, "z requires dz and out_ungated (the forward's ungated output)");
  const size_t need = ssm_scan_bwd_workspace_bytes(batch, dim, seqlen, nstate);
  if (!workspace || workspace_bytes < need)
    return fail(SSM_ERR_INVALID, "workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
  if (bc_batch_stride != 0 && bc_batch_stride < nstate * seqlen)
    return fail(SSM_ERR_INVALID, "bc_batch_stride must be 0 (contiguous) or at least nstate * seqlen (got %lld)",
                (long long)bc_batch_stride);
  ssm::ScanParams p = make_scan_params(batch, dim, seqlen, nstate, u, delta, A, B, C,
                                       bc_batch_stride, D, delta_bias,
                                       h_init, length, padding_right, z, delta_softplus);
  p.h_chunks_in = h_pairs ? h_chunks + dim : h_chunks;
  p.hs = h_pairs ? 2 : 1;
  if (h_pairs) p.nchunks = (int)(SSM_REF_SLOTS * ssm_scan_ref_nchunks(seqlen));
  p.dout = dout;
  p.dh_last = dh_last;
  p.du = du;
  p.ddelta = ddelta;
  p.dz = dz;
  p.out_ungated = const_cast<void*>(out_ungated);
  p.dh_init = dh_init;
  p.dA = dA;
  p.dB = dB;
  p.dC = dC;
  p.dD = dD;
  p.dbias = ddelta_bias;
  // workspace: [prepped B/C][dB/dC partials][dA partials][dD partials][dbias partials]
  // [segment carries and step sums][dummy]; the dA/dD/dbias partials have one
  // row per (segment, batch row)
  ssm::fwd_segments((int)batch, p.nblk, (int)seqlen, p.nseg, p.seg_len);
  // the role-split segment summaries split segments as the forward's do (the
  // carries fit the same workspace range)
  p.sub_k = ssm::fwd_summary_split((int)batch, p.nblk, p.nseg, p.seg_len);
  const size_t rows = (size_t)batch * p.nseg;
  char* ws = static_cast<char*>(workspace);
  float* bc = reinterpret_cast<float*>(ws);
  ws += round256(ssm::bc_prep_floats((int)batch, (int)nstate, (int)seqlen) * sizeof(float));
  p.ws_bc = reinterpret_cast<float*>(ws);
  ws += round256(2 * (size_t)p.nblk * batch * nstate * bwd_part_len(seqlen) * sizeof(float));
  p.ws_A = reinterpret_cast<float*>(ws);
  ws += round256(rows * dim * nstate * sizeof(float));
  p.ws_D = reinterpret_cast<float*>(ws);
  ws += round256(rows * dim * sizeof(float));
  p.ws_bias = reinterpret_cast<float*>(ws);
  ws += round256(rows * dim * sizeof(float));
  p.seg_h = reinterpret_cast<float*>(ws);
  p.seg_dt = p.seg_h + (size_t)(p.nseg - 1) * p.sub_k * batch * nstate * dim;
  ws += round256(ssm::fwd_seg_floats((int)batch, (int)dim, (int)nstate, (int)seqlen) * sizeof(float));
  p.nsc = (int)bwd_chunks(nstate);
  const size_t part_bytes = round256(p.nsc * (size_t)batch * dim * seqlen * sizeof(float));
  p.ws_gb = p.nsc ? reinterpret_cast<float*>(ws) : nullptr;
  p.ws_gd = p.nsc ? reinterpret_cast<float*>(ws + part_bytes) : nullptr;
  ws += 2 * part_bytes;
  p.dummy = ws;
  const bool aligned = scan_aligned(dtype, seqlen, {u, delta, z, out_ungated, dout, du, ddelta, dz});
  return hip_status(ssm::launch_scan_bwd(p, dtype, aligned, bc, static_cast<hipStream_t>(stream)),
                    "selective_scan backward launch");
}

int ssm_selective_scan_fwd_noalloc(int64_t batch, int64_t dim, int64_t seqlen, int64_t nstate,
                                   int dtype, const void* u, const void* delta, const float* A,
                                   const void* B, const void* C, int64_t bc_batch_stride,
                                   const float* D, const float* delta_bias, const float* h_init,
                                   const int64_t* length, int padding_right, const void* z,
                                   int delta_softplus, void* out, void* out_ungated,
                                   float* h_chunks, int h_pairs, float* h_last, void* stream) {
  g_err.clear();
  if (int e = check_common(batch, dim, seqlen, nstate, dtype, 256)) return e;
  const size_t need = ssm_scan_fwd_workspace_bytes(batch, dim, seqlen, nstate);
  if (need > (size_t)SSM_NOALLOC_SCRATCH_BYTES)
    return fail(SSM_ERR_UNSUPPORTED,
                "selective_scan forward without allocation: this shape needs %zu bytes of "
                "workspace, more than the %zu-byte static scratch (use ssm_selective_scan_fwd "
                "with a caller workspace)",
                need, (size_t)SSM_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (int e = scratch_on_current_device(&ws)) return e;
  // every workspace byte the kernels read is written by this call first
  // (prepped B/C, segment summaries), so nothing needs clearing
  return ssm_selective_scan_fwd(batch, dim, seqlen, nstate, dtype, u, delta, A, B, C,
                                bc_batch_stride, D, delta_bias, h_init, length, padding_right, z,
                                delta_softplus, out, out_ungated, h_chunks, h_pairs, h_last, ws,
                                (size_t)SSM_NOALLOC_SCRATCH_BYTES, stream);
}

namespace {
// Shape conditions of ssm_selective_scan_fwd_dt_proj (pointer conditions are
// checked by the entry point).
int check_dt_proj(int64_t batch, int64_t dim, int64_t seqlen, int64_t nstate, int64_t dt_rank,
                  int dtype) {
  if (int e = check_common(batch, dim, seqlen, nstate, dtype, 16)) return e;
  if (dtype != SSM_BF16)
    return fail(SSM_ERR_UNSUPPORTED, "the fused step-size projection takes bf16 only");
  if (dt_rank < 1) return fail(SSM_ERR_INVALID, "dt_rank must be >= 1 (got %lld)", (long long)dt_rank);
  if (dt_rank % 8 || dt_rank > 32 * ssm::kDtK)
    return fail(SSM_ERR_UNSUPPORTED, "the fused step-size projection takes dt_rank a multiple of 8 "
                "and <= %d (got %lld)", 32 * ssm::kDtK, (long long)dt_rank);
  if (nstate % 4)
    return fail(SSM_ERR_UNSUPPORTED, "the fused step-size projection takes nstate a multiple of 4 "
                "(16-byte token rows; got %lld)", (long long)nstate);
  const int64_t P = dt_rank + 2 * nstate;
  if (seqlen * P * 2 >= ((int64_t)1 << 31))
    return fail(SSM_ERR_UNSUPPORTED, "seqlen * (dt_rank + 2 nstate) * 2 bytes must be < 2^31");
  ssm::ScanParams p{};
  p.batch = (int)batch;
  p.dim = (int)dim;
  p.seqlen = (int)seqlen;
  p.nstate = (int)nstate;
  p.hs = 1;
  if (!ssm::scan_fwd_dt_supported(p))
    return fail(SSM_ERR_UNSUPPORTED, "the fused step-size projection: shape past the role-split "
                "kernel's buffer ranges");
  return SSM_OK;
}
}  // namespace

int ssm_selective_scan_fwd_dt_proj_supported(int64_t batch, int64_t dim, int64_t seqlen,
                                             int64_t nstate, int64_t dt_rank, int dtype) {
  const std::string keep = g_err;
  const int ok = check_dt_proj(batch, dim, seqlen, nstate, dt_rank, dtype) == SSM_OK;
  g_err = keep;
  return ok;
}

int ssm_selective_scan_fwd_dt_proj(int64_t batch, int64_t dim, int64_t seqlen, int64_t nstate,
                                   int64_t dt_rank, int dtype, const void* u,
                                   const void* ssm_params, int64_t params_batch_stride,
                                   const void* dt_weight, const float* A, const float* D,
                                   const float* delta_bias, const float* h_init,
                                   const int64_t* length, int padding_right, const void* z,
                                   int64_t z_batch_stride, int delta_softplus, void* out,
                                   void* delta_out, float* h_last, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  g_err.clear();
  if (int e = check_dt_proj(batch, dim, seqlen, nstate, dt_rank, dtype)) return e;
  if (!u || !ssm_params || !dt_weight || !A || !out)
    return fail(SSM_ERR_INVALID, "u, ssm_params, dt_weight, A and out must be non-NULL");
  const int64_t P = dt_rank + 2 * nstate;
  if (params_batch_stride != 0 && params_batch_stride < seqlen * P)
    return fail(SSM_ERR_INVALID, "params_batch_stride must be 0 (contiguous) or at least seqlen * "
                "(dt_rank + 2 nstate) (got %lld)", (long long)params_batch_stride);
  if (!aligned16(ssm_params) || !aligned16(dt_weight) || params_batch_stride % 8)
    return fail(SSM_ERR_UNSUPPORTED, "the fused step-size projection needs 16-byte aligned "
                "ssm_params rows and dt_weight");
  if (z_batch_stride != 0 && z_batch_stride < dim * seqlen)
    return fail(SSM_ERR_INVALID, "z_batch_stride must be 0 (contiguous) or at least dim * seqlen "
                "(got %lld)", (long long)z_batch_stride);
  const size_t need = ssm_scan_fwd_workspace_bytes(batch, dim, seqlen, nstate);
  if (!workspace || workspace_bytes < need)
    return fail(SSM_ERR_INVALID, "workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
  ssm::ScanParams p = make_scan_params(batch, dim, seqlen, nstate, u, u, A, ssm_params, ssm_params,
                                       0, D, delta_bias, h_init, length, padding_right, z,
                                       delta_softplus);
  p.out = out;
  p.hs = 1;
  p.h_last = h_last;
  // workspace: [prepped B/C (unused here)][segment states and step sums][dummy]
  char* ws = static_cast<char*>(workspace) +
             round256(ssm::bc_prep_floats((int)batch, (int)nstate, (int)seqlen) * sizeof(float));
  ssm::fwd_segments((int)batch, p.nblk, (int)seqlen, p.nseg, p.seg_len);
  p.sub_k = ssm::fwd_summary_split((int)batch, p.nblk, p.nseg, p.seg_len);
  p.seg_h = reinterpret_cast<float*>(ws);
  p.seg_dt = p.seg_h + (size_t)(p.nseg - 1) * p.sub_k * batch * nstate * dim;
  ws += round256(ssm::fwd_seg_floats((int)batch, (int)dim, (int)nstate, (int)seqlen) * sizeof(float));
  p.dummy = ws;
  ssm::DtProj dt{};
  dt.params = ssm_params;
  dt.pstride = params_batch_stride ? params_batch_stride : seqlen * P;
  dt.P = (int)P;
  dt.rank = (int)dt_rank;
  dt.w = dt_weight;
  dt.delta_out = delta_out;
  dt.zbstride = z_batch_stride ? z_batch_stride : dim * seqlen;
  const bool aligned = scan_aligned(dtype, seqlen, {u, z, out}) && dt.zbstride % 8 == 0;
  return hip_status(ssm::launch_scan_fwd_dt(p, dt, aligned, static_cast<hipStream_t>(stream)),
                    "selective_scan forward with the step-size projection launch");
}

int ssm_selective_state_update(int64_t batch, int64_t dim, int64_t nstate, int dtype,
                               const float* state, float* new_state, const void* x,
                               const void* dt, const float* A, const void* B, const void* C,
                               const float* D, const float* dt_bias, const void* z,
                               int dt_softplus, void* out, void* stream) {
  g_err.clear();
  if (int e = check_common(batch, dim, 1, nstate, dtype, 256)) return e;
  if (dim * 64 > INT_MAX || batch * dim * nstate >= ((int64_t)1 << 31))
    return fail(SSM_ERR_UNSUPPORTED, "state too large: batch * dim * nstate must be < 2^31");
  if (!state || !new_state || !x || !dt || !A || !B || !C || !out)
    return fail(SSM_ERR_INVALID, "state, new_state, x, dt, A, B, C and out must be non-NULL");
  ssm::UpdateParams p{};
  p.batch = (int)batch;
  p.dim = (int)dim;
  p.nstate = (int)nstate;
  p.softplus = dt_softplus ? 1 : 0;
  p.state = state;
  p.new_state = new_state;
  p.x = x;
  p.dt = dt;
  p.A = A;
  p.B = B;
  p.C = C;
  p.D = D;
  p.bias = dt_bias;
  p.z = z;
  p.out = out;
  // 128-bit path: N in {4, 8, 16, 32, 64} with 16-byte aligned state / A and
  // 8-byte (bf16) or 16-byte (fp32) aligned B / C rows
  const bool vecN = nstate % 4 == 0 && aligned16(state) && aligned16(new_state) && aligned16(A) &&
                    (dtype == SSM_F32 ? aligned16(B) && aligned16(C)
                                      : (((uintptr_t)B | (uintptr_t)C) & 7) == 0);
  return hip_status(ssm::launch_state_update(p, dtype, vecN, static_cast<hipStream_t>(stream)),
                    "selective_state_update launch");
}

int ssm_decode_gemv(int64_t batch, int64_t out_dim, int64_t in_dim, int dtype, const void* weight,
                    const void* x, const void* norm_weight, float norm_eps, const void* bias,
                    const void* residual, void* y, void* stream) {
  int rc = check_decode(batch, dtype);
  if (rc != SSM_OK) return rc;
  if (!weight || !x || !y) return fail(SSM_ERR_INVALID, "weight, x and y must be non-NULL");
  const int e = elems16(dtype);
  if (out_dim < 1 || in_dim < e || in_dim % e || out_dim > INT_MAX / 2 || in_dim > INT_MAX / 2)
    return fail(SSM_ERR_UNSUPPORTED, "decode_gemv needs in_dim a positive multiple of %d (got %lld x %lld)",
                e, (long long)out_dim, (long long)in_dim);
  if (!aligned16(weight) || !aligned16(x) || !aligned16(norm_weight))
    return fail(SSM_ERR_UNSUPPORTED, "decode_gemv needs 16-byte aligned weight, x and norm_weight");
  return hip_status(ssm::launch_decode_gemv(dtype == SSM_BF16, weight, x, norm_weight, norm_eps, bias,
                                            residual, y, (int)batch, (int)out_dim, (int)in_dim,
                                            static_cast<hipStream_t>(stream)),
                    "decode_gemv launch");
}

int64_t ssm_decode_xproj_blocks(int64_t dim, int64_t params_dim) {
  return ssm::decode_xproj_blocks(dim, params_dim);
}

int ssm_decode_in_proj_conv(int64_t batch, int64_t dim, int64_t in_dim, int64_t width, int dtype,
                            const void* in_proj_weight, const void* x, const void* norm_weight,
                            float norm_eps, const void* in_proj_bias, const void* conv_weight,
                            const void* conv_bias, void* conv_window, void* xz, void* xc,
                            const void* x_proj_weight, int64_t params_dim, float* xproj_partials,
                            void* stream) {
  int rc = check_decode(batch, dtype);
  if (rc != SSM_OK) return rc;
  if (!in_proj_weight || !x || !conv_weight || !conv_window || !xz || !xc)
    return fail(SSM_ERR_INVALID,
                "in_proj_weight, x, conv_weight, conv_window, xz and xc must be non-NULL");
  const int e = elems16(dtype);
  if (in_dim < e || in_dim % e || in_dim > INT_MAX / 2)
    return fail(SSM_ERR_UNSUPPORTED, "decode_in_proj_conv needs in_dim a positive multiple of %d", e);
  if (dim < 1 || dim > INT_MAX / 4)
    return fail(SSM_ERR_UNSUPPORTED, "decode_in_proj_conv needs 1 <= dim < 2^29");
  if (width < 2 || width > ssm::conv1d_max_width())
    return fail(SSM_ERR_UNSUPPORTED, "decode conv width must be in [2, %d] (got %lld)",
                ssm::conv1d_max_width(), (long long)width);
  if (!aligned16(in_proj_weight) || !aligned16(x) || !aligned16(norm_weight))
    return fail(SSM_ERR_UNSUPPORTED, "decode_in_proj_conv needs 16-byte aligned weight, x and norm_weight");
  if ((x_proj_weight != nullptr) != (xproj_partials != nullptr))
    return fail(SSM_ERR_INVALID, "x_proj_weight and xproj_partials go together");
  if (x_proj_weight) {
    if (ssm::decode_xproj_blocks(dim, params_dim) == 0)
      return fail(SSM_ERR_UNSUPPORTED,
                  "the folded x-projection needs ssm_decode_xproj_blocks(dim, params_dim) > 0 "
                  "(got dim %lld, params_dim %lld)", (long long)dim, (long long)params_dim);
    if (!aligned16(x_proj_weight) || !aligned16(xproj_partials))
      return fail(SSM_ERR_UNSUPPORTED, "decode_in_proj_conv needs 16-byte aligned x_proj_weight and xproj_partials");
  }
  return hip_status(ssm::launch_decode_in_proj_conv(dtype == SSM_BF16, in_proj_weight, x, norm_weight,
                                                    norm_eps, in_proj_bias, xz, (int)batch, (int)dim,
                                                    (int)in_dim, (int)width, conv_window, conv_weight,
                                                    conv_bias, xc, x_proj_weight,
                                                    x_proj_weight ? (int)params_dim : 0, xproj_partials,
                                                    static_cast<hipStream_t>(stream)),
                    "decode_in_proj_conv launch");
}

int ssm_decode_ssm_step(int64_t batch, int64_t dim, int64_t nstate, int64_t rank, int dtype,
                        const void* params, int64_t params_blocks, const void* dt_proj_weight,
                        const void* dt_bias, const void* log_A, const void* D, const void* xc,
                        const void* xz, int64_t ld_xz, float* state, void* y, void* stream) {
  int rc = check_decode(batch, dtype);
  if (rc != SSM_OK) return rc;
  if (!params || !dt_proj_weight || !log_A || !xc || !xz || !state || !y)
    return fail(SSM_ERR_INVALID, "params, dt_proj_weight, log_A, xc, xz, state and y must be non-NULL");
  if (!(nstate == 4 || nstate == 8 || nstate == 16 || nstate == 32 || nstate == 64))
    return fail(SSM_ERR_UNSUPPORTED, "decode_ssm_step supports nstate in {4, 8, 16, 32, 64} (got %lld)",
                (long long)nstate);
  const int64_t nout = rank + 2 * nstate;
  if (dim < 1 || dim > INT_MAX / 4 || rank < 1 || nout > 16384 || ld_xz < 2 * dim)
    return fail(SSM_ERR_UNSUPPORTED,
                "decode_ssm_step needs dim >= 1, rank >= 1, rank + 2 * nstate <= 16384, ld_xz >= 2 * dim");
  if (!aligned16(state)) return fail(SSM_ERR_UNSUPPORTED, "decode_ssm_step needs a 16-byte aligned state");
  if (params_blocks) {
    if (params_blocks != ssm::decode_xproj_blocks(dim, nout))
      return fail(SSM_ERR_INVALID, "params_blocks must be 0 or ssm_decode_xproj_blocks(dim, rank + 2 * nstate) = %d (got %lld)",
                  ssm::decode_xproj_blocks(dim, nout), (long long)params_blocks);
    if (!aligned16(params))
      return fail(SSM_ERR_UNSUPPORTED, "decode_ssm_step needs 16-byte aligned x-projection partials");
  }
  const bool vecR = rank % elems16(dtype) == 0 && rank <= 16 * elems16(dtype) &&
                    aligned16(dt_proj_weight);
  return hip_status(ssm::launch_decode_ssm_step(dtype == SSM_BF16, params, (int)nout,
                                                (int)params_blocks, (int)rank,
                                                dt_proj_weight, dt_bias, log_A, D, xc, xz, (int)ld_xz,
                                                state, y, (int)batch, (int)dim, (int)nstate, vecR,
                                                static_cast<hipStream_t>(stream)),
                    "decode_ssm_step launch");
}

int64_t ssm_decode_layers_workspace(int64_t batch, int64_t nlayers, int64_t model_dim, int64_t dim,
                                    int64_t params_dim, int dtype) {
  if (check_decode(batch, dtype) != SSM_OK || nlayers < 1 || nlayers > 65536 || model_dim < 1 ||
      model_dim > INT_MAX / 16 || ssm::decode_xproj_blocks(dim, params_dim) == 0)
    return 0;
  return ssm::decode_layers_workspace((int)batch, (int)nlayers, (int)model_dim, (int)dim,
                                      (int)params_dim, dtype == SSM_BF16);
}

int ssm_decode_layers(int64_t batch, int64_t nlayers, int64_t model_dim, int64_t dim, int64_t nstate,
                      int64_t rank, int64_t width, int dtype, const void* layer_table, const void* x,
                      void* out, float norm_eps, void* workspace, int64_t workspace_bytes,
                      void* stream) {
  int rc = check_decode(batch, dtype);
  if (rc != SSM_OK) return rc;
  if (!layer_table || !x || !out || !workspace)
    return fail(SSM_ERR_INVALID, "layer_table, x, out and workspace must be non-NULL");
  if (nlayers < 1 || nlayers > 65536)
    return fail(SSM_ERR_INVALID, "decode_layers needs 1 <= nlayers <= 65536 (got %lld)", (long long)nlayers);
  if (nstate != 16)
    return fail(SSM_ERR_UNSUPPORTED, "decode_layers supports nstate 16 (got %lld)", (long long)nstate);
  const int e = elems16(dtype);
  if (model_dim < e || model_dim % e || model_dim > INT_MAX / 16)
    return fail(SSM_ERR_UNSUPPORTED, "decode_layers needs model_dim a positive multiple of %d", e);
  if (rank < 1 || rank % e || rank > 8 * e)
    return fail(SSM_ERR_UNSUPPORTED, "decode_layers needs rank a multiple of %d and at most %d (got %lld)",
                e, 8 * e, (long long)rank);
  const int64_t nout = rank + 2 * nstate;
  if (dim > (1 << 24) || ssm::decode_xproj_blocks(dim, nout) == 0)
    return fail(SSM_ERR_UNSUPPORTED,
                "decode_layers needs the folded x-projection: ssm_decode_xproj_blocks(dim, rank + 2 * nstate) > 0");
  if (width < 2 || width > ssm::decode_layers_max_width())
    return fail(SSM_ERR_UNSUPPORTED, "decode_layers conv width must be in [2, %d] (got %lld)",
                ssm::decode_layers_max_width(), (long long)width);
  if (const char* why = ssm::decode_layers_unsupported((int)model_dim, (int)dim, (int)nout,
                                                       dtype == SSM_BF16))
    return fail(SSM_ERR_UNSUPPORTED, "decode_layers: %s (model_dim %lld, dim %lld, params_dim %lld)",
                why, (long long)model_dim, (long long)dim, (long long)nout);
  if (!aligned16(x) || !aligned16(out) || (reinterpret_cast<uintptr_t>(workspace) & 255) ||
      (reinterpret_cast<uintptr_t>(layer_table) & 7))
    return fail(SSM_ERR_UNSUPPORTED,
                "decode_layers needs 16-byte aligned x and out, a 256-byte aligned workspace and an 8-byte aligned layer_table");
  const int64_t need = ssm::decode_layers_workspace((int)batch, (int)nlayers, (int)model_dim,
                                                    (int)dim, (int)nout, dtype == SSM_BF16);
  if (workspace_bytes < need)
    return fail(SSM_ERR_INVALID, "decode_layers workspace is %lld bytes, needs %lld",
                (long long)workspace_bytes, (long long)need);
  const hipError_t he = ssm::launch_decode_layers(dtype == SSM_BF16, layer_table, (int)nlayers,
                                                  (int)batch, (int)model_dim, (int)dim, (int)width,
                                                  (int)rank, (int)nout, norm_eps, x, out, workspace,
                                                  static_cast<hipStream_t>(stream));
  if (he == hipErrorCooperativeLaunchTooLarge)
    return fail(SSM_ERR_UNSUPPORTED,
                "decode_layers needs all %d workgroups resident at once, more than this device holds",
                ssm::decode_layers_grid((int)batch, (int)model_dim, (int)dim));
  return hip_status(he, "decode_layers launch");
}

int64_t ssm_decode_pick_workspace(int64_t batch) {
  return batch < 1 || batch > ssm::decode_max_batch() ? 0 : ssm::decode_pick_workspace((int)batch);
}

int ssm_decode_pick(int64_t batch, int64_t vocab, int dtype, const void* probs, int64_t* token,
                    int64_t* tokens, int64_t tokens_ld, int64_t tokens_cols, int64_t* pos,
                    void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = check_decode(batch, dtype);
  if (rc != SSM_OK) return rc;
  if (!probs || !token || !workspace) return fail(SSM_ERR_INVALID, "probs, token and workspace must be non-NULL");
  if (workspace_bytes < ssm::decode_pick_workspace((int)batch))
    return fail(SSM_ERR_INVALID, "decode_pick workspace is %lld bytes, needs %lld",
                (long long)workspace_bytes, (long long)ssm::decode_pick_workspace((int)batch));
  if (vocab < 1 || vocab > INT_MAX / 2)
    return fail(SSM_ERR_INVALID, "decode_pick needs 1 <= vocab < 2^30 (got %lld)", (long long)vocab);
  if (tokens && (tokens_cols < 1 || tokens_ld < tokens_cols))
    return fail(SSM_ERR_INVALID, "decode_pick needs tokens_cols >= 1 and tokens_ld >= tokens_cols");
  if (!aligned16(probs) || (vocab * (dtype == SSM_BF16 ? 2 : 4)) % 16)
    return fail(SSM_ERR_UNSUPPORTED, "decode_pick needs 16-byte aligned rows (vocab %lld)",
                (long long)vocab);
  return hip_status(ssm::launch_decode_pick(dtype == SSM_BF16, probs, (int)batch, (int)vocab, token,
                                            tokens, tokens_ld, tokens ? tokens_cols : 1, pos,
                                            workspace, static_cast<hipStream_t>(stream)),
                    "decode_pick launch");
}

int ssm_decode_layers_status(void* workspace, int64_t workspace_bytes, void* stream) {
  if (!workspace || workspace_bytes < ssm::decode_layers_error_offset() + 4)
    return fail(SSM_ERR_INVALID, "workspace must be non-NULL and hold at least the sync area");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  unsigned err = 0;
  // the error word of the sync area at the start of the workspace
  const char* word = static_cast<const char*>(workspace) + ssm::decode_layers_error_offset();
  if (int rc = hip_status(hipMemcpyAsync(&err, word, sizeof(err), hipMemcpyDeviceToHost, st),
                          "decode_layers status copy"))
    return rc;
  if (int rc = hip_status(hipStreamSynchronize(st), "decode_layers status sync")) return rc;
  if (!err) return SSM_OK;
  if (int rc = hip_status(hipMemsetAsync(workspace, 0, (size_t)workspace_bytes, st),
                          "decode_layers workspace reset"))
    return rc;
  if (int rc = hip_status(hipStreamSynchronize(st), "decode_layers workspace reset")) return rc;
  return fail(SSM_ERR_HIP,
              "decode_layers: a wait for another workgroup's data timed out (not every workgroup "
              "was resident); the outputs of the launches since the last status check are "
              "invalid, and so are the layers' SSM states and conv windows, which those launches "
              "may have advanced in part (re-run the prefill); the workspace is cleared");
}

int ssm_rms_norm_cm(int64_t batch, int64_t channels, int64_t seqlen, int dtype, const void* x,
                    const void* weight, float eps, void* out, void* stream) {
  if (dtype != SSM_F32 && dtype != SSM_BF16)
    return fail(SSM_ERR_INVALID, "dtype must be SSM_F32 or SSM_BF16 (got %d)", dtype);
  if (batch < 1 || channels < 1 || seqlen < 1)
    return fail(SSM_ERR_INVALID, "batch, channels and seqlen must be >= 1");
  if (channels > INT_MAX / 2 || seqlen > INT_MAX / 2 || batch * ((seqlen + 127) / 128) > INT_MAX)
    return fail(SSM_ERR_UNSUPPORTED, "rms_norm_cm sizes too large");
  if (!x || !weight || !out) return fail(SSM_ERR_INVALID, "x, weight and out must be non-NULL");
  const uintptr_t align = dtype == SSM_BF16 ? 4 : 8;
  const bool pair = seqlen % 2 == 0 && ((uintptr_t)x % align) == 0 && ((uintptr_t)out % align) == 0;
  return hip_status(ssm::launch_rms_norm_cm(dtype == SSM_BF16, x, weight, eps, out, (int)batch,
                                            (int)channels, (int)seqlen, pair,
                                            static_cast<hipStream_t>(stream)),
                    "rms_norm_cm launch");
}

size_t ssm_causal_conv1d_bwd_workspace_bytes(int64_t batch, int64_t dim, int64_t width) {
  if (batch < 1 || dim < 1 || width < 1) return 0;
  return round256((size_t)batch * (size_t)dim * (size_t)(width + 1) * sizeof(float));
}

int ssm_causal_conv1d_fwd(int64_t batch, int64_t dim, int64_t seqlen, int64_t width, int dtype,
                          const void* x, int64_t x_batch_stride, const void* weight,
                          const void* bias, int silu, void* out, const int64_t* lengths,
                          void* window, void* stream) {
  int rc = check_conv(batch, dim, seqlen, width, dtype);
  if (rc != SSM_OK) return rc;
  if (!x || !weight || !out) return fail(SSM_ERR_INVALID, "x, weight and out must be non-NULL");
  if (lengths && !window) return fail(SSM_ERR_INVALID, "lengths requires window");
  if (x_batch_stride != 0 && x_batch_stride < dim * seqlen)
    return fail(SSM_ERR_INVALID, "x_batch_stride must be 0 (contiguous) or at least dim * seqlen "
                "(got %lld)", (long long)x_batch_stride);
  const int64_t xbs = x_batch_stride ? x_batch_stride : dim * seqlen;
  const bool vec = seqlen % 8 == 0 && xbs % 8 == 0 && aligned16(x) && aligned16(out);
  return hip_status(ssm::launch_causal_conv1d_fwd((int)batch, (int)dim, (int)seqlen, (int)width,
                                                  dtype == SSM_BF16, x, xbs, weight, bias,
                                                  silu ? 1 : 0, out, lengths, window, vec,
                                                  static_cast<hipStream_t>(stream)),
                    "causal_conv1d_fwd launch");
}

int ssm_causal_conv1d_bwd(int64_t batch, int64_t dim, int64_t seqlen, int64_t width, int dtype,
                          const void* x, const void* weight, const void* bias, const void* dout,
                          int silu, void* dx, void* dweight, void* dbias, void* workspace,
                          size_t workspace_bytes, void* stream) {
  int rc = check_conv(batch, dim, seqlen, width, dtype);
  if (rc != SSM_OK) return rc;
  if (!x || !weight || !dout || !dx || !dweight)
    return fail(SSM_ERR_INVALID, "x, weight, dout, dx and dweight must be non-NULL");
  const size_t need = ssm_causal_conv1d_bwd_workspace_bytes(batch, dim, width);
  if (!workspace || workspace_bytes < need)
    return fail(SSM_ERR_INVALID, "workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
  const bool vec = seqlen % 8 == 0 && aligned16(x) && aligned16(dout) && aligned16(dx);
  return hip_status(ssm::launch_causal_conv1d_bwd((int)batch, (int)dim, (int)seqlen, (int)width,
                                                  dtype == SSM_BF16, x, weight, bias, dout,
                                                  silu ? 1 : 0, dx, dweight, dbias,
                                                  static_cast<float*>(workspace), vec,
                                                  static_cast<hipStream_t>(stream)),
                    "causal_conv1d_bwd launch");
}

}  // extern "C"
