// g4v_capi.hip -- the C ABI (include/g4v.h): context, uploads, the standalone kernel entry
// points and the verify-step orchestration that restates the reference's fwd()/run_req.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <functional>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/g4v.h"
#include "g4v_head.h"
#include "g4v_internal.h"
#include "g4v_layer.h"

using namespace g4v;

namespace {

struct DBuf {
  void* p = nullptr;
  size_t n = 0;
  DBuf() = default;
  DBuf(const DBuf&) = delete;
  DBuf& operator=(const DBuf&) = delete;
  ~DBuf() { reset(); }
  void reset() {
    if (p) (void)hipFree(p);
    p = nullptr;
    n = 0;
  }
  template <class T>
  T* as() const { return static_cast<T*>(p); }
};

struct Mat {
  DBuf wr, s;
  DBuf tw, ts;  // row-tiled copies for the row-tile GEMV (verify-pass q, k, v, o, down; the gate
                // matrix holds the gate / up pair)
  DBuf a8w, a8s;  // W4A8 MFMA operand tiles (standalone handles with N % 16 == 0)
  int N = 0, K = 0;
  W4Dev dev() const { return W4Dev{wr.as<uint4>(), s.as<uint16_t>(), N, K}; }
  W4Tile tile() const { return W4Tile{tw.as<uint4>(), ts.as<uint4>(), N}; }
};

// the layer matrices the verify pass multiplies with the row-tile GEMV: q, k, v, o, down (gate
// and up as one pair, tile_gateup)
static bool row_tiled(int j) { return j <= 3 || j == 6; }

struct Layer {
  Mat m[7];       // q, k, v, o, gate, up, down
  DBuf norms;     // in_ln, post_attn, pre_ff, post_ff [H each], qn, kn [HD each], qn, kn in the
                  // 16-lane head order [HD each] (head16_index; refreshed by perm_norms)
  float scalar = 0.75f;
  int sliding = 1;
  LayerNorms ln() const {
    const float* b = norms.as<float>();
    return LayerNorms{b,           b + H, b + 2 * H, b + 3 * H, b + 4 * H, b + 4 * H + HD, b + 4 * H + 2 * HD,
                      b + 4 * H + 3 * HD, scalar, sliding};
  }
  // the q / k norm weights' copies in the attention's 16-lane order, after a write of the norms
  void perm_norms(hipStream_t st) const {
    const float* b = norms.as<float>();
    float* d = const_cast<float*>(b) + 4 * H + 2 * HD;
    launch_perm16(b + 4 * H, d, st);
    launch_perm16(b + 4 * H + HD, d + HD, st);
  }
};

// scratch of one head pass
struct HeadBufs {
  DBuf u, list, sval, small, part;
  HeadScratch hs{};
};

}  // namespace

struct g4v_ctx {
  int device = 0;
  hipStream_t st = nullptr;
  std::string err;
  int lds_max = 65536;
  int cus = 0;
  std::vector<std::unique_ptr<Mat>> mats;  // standalone GEMV handles
  DBuf gx, gy;                              // standalone GEMV io
  DBuf nrmio;                               // g4v_w4g32_norm_gemm io: o, xin, x1 [MAXM][H], w1, w2 [H]
  DBuf a8x, a8y, a8xq, a8sx, a8corr, a8q, a8qs, a8qsum;  // W4A8 io and quantised activations
  // head
  bool head_ready = false;
  int V = 0;
  DBuf E, dec, x3sm, x3ix, exc_ptr, exc_col, exc_del, cb, scr_wr, scr_s, coef, lut;
  HeadDev hd{};
  HeadBufs hb1, hb2;
  DBuf hrow, hnrow;
  // model
  bool model_ready = false;  // buffers allocated (model_synth or model_create)
  int NL = 0, I = 0, ctxcap = 0, kvcap = 0;  // kvcap: positions per layer slab of the KV cache
  std::vector<std::unique_ptr<Layer>> L;
  DBuf fnorm, KC, VC, rope;  // rope: [2 types][cos, sin][ctxcap][HD/2]
  DBuf ropestep;             // the step's rows of it: [2 types][MAXM][cos | sin][HD/2]
  // step buffers
  // xa and act hold GEMV inputs in the staged layout (staged_index), xgs the group sums of xa
  // x / x2: the residual stream, alternating between the two halves of a layer (a GEMV whose
  // norm prologue updates it reads one and writes the other)
  DBuf x, x2, xa, xgs, q, k, v, o, act, h, hn, h2, hn2, po, pm, pl, stepd, resd;
  DBuf vatt, vsc;  // a pass's attn_tile / run_mh output (staged) and its score scratch
  StepDev* step_host = nullptr;
  VerifyResultDev* res_host = nullptr;
  // attention standalone
  DBuf ak, av, aq, ao;
  DBuf vags;  // group sums of the merged attention rows of a W4A8 verify pass [MAXM][NQ * HD / 32]
  // W4A8 verify passes: the rows of the next product quantised by their producer (the split-KV
  // merge for o, the 6144-wide gate / up for down): operand words [MAXM][384][4], scales [MAXM][384]
  DBuf q8w, q8s;
  DBuf po5, pm5, pl5;  // split partials at head dim 512
  // the Gemma-4-E2B layout (g4v_model_create_gemma): per-layer geometry, the per-layer-input
  // branch, the owners' caches and the row buffers of its passes
  bool gemma = false;
  struct GmLayer {
    int hd = 256, own = 1, I = 0;
    Mat pg, pp;   // per_layer_input_gate [256][1536], per_layer_projection [1536][256]
    DBuf nv;      // in_ln, post_attn, pre_ff, post_ff, post_ple [1536 each], qn, kn [hd each]
    float scalar = 1.0f;
    bool normed = false;
  };
  GmLayer gm[35];
  Mat gm_plproj;                  // per_layer_model_projection [8960][1536]
  DBuf gm_plnorm, gm_ple;         // per_layer_projection_norm [256]; the table [V][8960] bf16
  DBuf gm_kv;                     // layer l < 15: K at gm_koff[l], V at gm_voff[l], [kvcap][hd] each
  size_t gm_koff[15] = {}, gm_voff[15] = {};
  DBuf gm_rope;                   // global layers' RoPE: cos, sin [ctxcap][256]
  DBuf gm_rows, gm_tok, gm_s;     // row buffers of a pass (gm_cap rows), its tokens, score scratch
  DBuf gm_geo;                    // a verify pass's split geometry per layer type (launch_step_geom)
  int gm_cap = 0;                 // rows the row buffers, tokens and W4A8 operands hold
  size_t gm_sfl = 0;              // floats of the score scratch
  int gm_Imax = 0;
  bool gm_plready = false;
  // prefill rows (plain [row][K] layouts), quantised activations, attention score scratch
  DBuf pfx, pfa, pfq, pfk, pfv, pfatt, pfo, pfg, pfu, pfact, pfxq, pfsx, pfcorr, pfs, pftok, pfh;
  int pf_rows = 0, pf_I = 0;  // rows and FFN width the buffers were sized for
  size_t pf_sfl = 0;
  // MTP drafter: tensors, then scratch of a chain (dx, da, y, q, att, act, dh, two hidden
  // states, centroid scores, candidates and their scores, tokens, runners-up, gaps)
  bool dr_ready = false;
  int dr_C = 0;
  int dr_hd[4] = {256, 256, 256, 256};  // layer head dims (the global layer 3: 256 synthetic, 512 loaded)
  float dr_scalar[4] = {0.75f, 0.75f, 0.75f, 0.75f};
  DBuf dr_pre, dr_post, dr_cent, dr_emb, dr_order, dr_norms, dr_q[4], dr_o[4], dr_g[4], dr_u[4], dr_d[4], dr_s;
  int last_hrow = -1;  // row of c->h holding the last verify step's committed hidden state
  int pf_nsurv = 0, pf_fallback = 0;  // the last prefill's head row: screen survivors, fallback
  int* dr_in_host = nullptr;   // pinned chain inputs {tok, P, hrow, _, h[1536]}
  int* dr_out_host = nullptr;  // pinned chain outputs {tok[8], sec[8], gap[8], hidden[1536]}
  // prefix cache: the active KV (KC / VC) with its keys, plus stored slots (each a full KV copy)
  struct Slot {
    DBuf KC, VC;
    std::vector<int> keys;
    int kv_len = 0;
    uint64_t stamp = 0;
  };
  std::vector<std::unique_ptr<Slot>> slots;
  std::vector<int> act_keys;
  int act_kv_len = 0, min_reuse = 32;
  uint64_t act_stamp = 0, clock_tick = 0;
  // prompt-lookup history (prompt + committed tokens) and the lookup's result words
  DBuf hist, plout;
  int hist_len = 0, hist_cap = 0;
  int* pl_host = nullptr;
  // per-kernel-class HIP-event timing on the library stream (g4v_profile)
  unsigned prof_mask = 0;
  std::vector<hipEvent_t> evpool;
  size_t evused = 0;
  struct Rec {
    int tag;
    hipEvent_t a, b;
    double bytes;
  };
  std::vector<Rec> recs;
  hipEvent_t open_ev = nullptr;
  double prof_ms[PT_NTAGS] = {0}, prof_bytes[PT_NTAGS] = {0};
  long long prof_n[PT_NTAGS] = {0};
  // captured verify steps, one per (rows, branches, splits, profile mask)
  struct Graph {
    long long key;
    hipGraphExec_t exec;
    std::vector<Rec> recs;          // profiling intervals baked into the graph
    std::vector<hipEvent_t> events; // owned
  };
  std::vector<Graph> graphs;
  std::vector<long long> warmed;  // shapes run once eagerly (first call) before capture
  bool use_graph = true;
  bool pf_i8 = true;  // G_I8 (ENGINE_PREFILL_INT8=1): prefill blocks of two rows or more run W4A8
  // ENGINE_DECODE_INT8 (E:1600): with pf_i8, the decode keeps G_I8_ACTIVE, so verify passes of
  // two rows or more run W4A8 too (Gemma layout)
  bool dec_i8 = false;
  bool dr_same = false;  // ENGINE_DRAFT_SAMEPOS (E:1516, 1633): every draft step at position P + 1
  // row-tile GEMV shape of the verify pass's q/k/v, o, gate/up and down products: activation
  // rows per block and rows per tile (G4V_GEMV_CFG="a,b a,b a,b a,b" overrides, for tuning)
  int gcfg[4][2] = {{2, 64}, {1, 64}, {4, 64}, {1, 64}};
  size_t step_events = 0;  // profiling events used by the last eager verify pass
  ~g4v_ctx() {
    for (auto& g : graphs) {
      (void)hipGraphExecDestroy(g.exec);
      for (hipEvent_t e : g.events) (void)hipEventDestroy(e);
    }
    for (hipEvent_t e : evpool) (void)hipEventDestroy(e);
    if (step_host) (void)hipHostFree(step_host);
    if (res_host) (void)hipHostFree(res_host);
    if (pl_host) (void)hipHostFree(pl_host);
    if (dr_in_host) (void)hipHostFree(dr_in_host);
    if (dr_out_host) (void)hipHostFree(dr_out_host);
    if (st) (void)hipStreamDestroy(st);
  }
};

#define HIPCHK(expr)                                                                       \
  do {                                                                                     \
    hipError_t e_ = (expr);                                                                \
    if (e_ != hipSuccess) {                                                                \
      c->err = std::string(#expr) + ": " + hipGetErrorString(e_);                          \
      return G4V_E_HIP;                                                                    \
    }                                                                                      \
  } while (0)

#define ARGCHK(cond, msg)        \
  do {                           \
    if (!(cond)) {               \
      c->err = msg;              \
      return G4V_E_ARG;          \
    }                            \
  } while (0)

static int dalloc(g4v_ctx* c, DBuf& b, size_t n) {
  b.reset();
  if (n == 0) n = 16;
  hipError_t e = hipMalloc(&b.p, n);
  if (e != hipSuccess) {
    b.p = nullptr;
    c->err = std::string("hipMalloc(") + std::to_string(n) + "): " + hipGetErrorString(e);
    return G4V_E_NOMEM;
  }
  b.n = n;
  return 0;
}
#define ALLOC(buf, n)                       \
  do {                                      \
    int r_ = dalloc(c, buf, (size_t)(n));   \
    if (r_) return r_;                      \
  } while (0)

// Captured graphs hold raw device pointers: every call that frees or reallocates model, head
// or step buffers must drop them first (a replay would touch freed memory).
static void drop_graphs(g4v_ctx* c) {
  (void)hipStreamSynchronize(c->st);
  for (auto& g : c->graphs) {
    (void)hipGraphExecDestroy(g.exec);
    for (hipEvent_t e : g.events) (void)hipEventDestroy(e);
  }
  c->graphs.clear();
  c->warmed.clear();
}

// profiling hook: brackets a launch (or a group of launches) of class `tag` with events
static void pmark(void* p, int tag, int begin, double bytes) {
  g4v_ctx* c = static_cast<g4v_ctx*>(p);
  if (!(c->prof_mask & (1u << tag))) return;
  if (c->evused == c->evpool.size()) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    (void)hipStreamIsCapturing(c->st, &cs);
    if (cs != hipStreamCaptureStatusNone) return;  // never create an event inside a capture
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return;
    c->evpool.push_back(e);
  }
  hipEvent_t e = c->evpool[c->evused++];
  (void)hipEventRecord(e, c->st);
  if (begin) c->open_ev = e;
  else c->recs.push_back({tag, c->open_ev, e, bytes});
}

// after the stream has drained: fold the recorded intervals into the per-class totals
static void prof_collect(g4v_ctx* c, bool full_ran) {
  for (const auto& r : c->recs) {
    float ms = 0;
    if (hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess) {
      (void)hipGetLastError();  // a failed timing query must not surface as a later launch error
      continue;
    }
    c->prof_ms[r.tag] += ms;
    c->prof_bytes[r.tag] += (r.tag == PT_HEAD_FULL && !full_ran) ? 0.0 : r.bytes;
    c->prof_n[r.tag] += 1;
  }
  c->recs.clear();
  c->evused = 0;
}

// GEMV over all M rows in one launch (the kernel stages K in phases when the activations
// of M rows exceed its LDS budget)
static void gemv_passes(g4v_ctx* c, GemvArgs a, int epi, int M) {
  a.M = M;
  launch_gemv(a, epi, c->st);
}

extern "C" {

// ---------------------------------------------------------------------------------------
// scratch of g4v_attn_splitkv_noalloc: a file-scope device array (each GPU holds its own copy
// until the process ends) with the caller's key and value rows in the device cache layout
// (NA_NPOS positions each) and the split partials po [MAXT][MAXM][NQ][HD], pm, pl [MAXT][MAXM][NQ].
// Host code never uses the array's name as an address: its device address is taken once per
// device with hipGetSymbolAddress (at the device's first g4v_create) and kept in na_scratch.
constexpr int NA_NPOS = 4096;
constexpr size_t NA_KV = (size_t)NA_NPOS * HD * 2;
constexpr size_t NA_PO = (size_t)MAXT * MAXM * NQ * HD * 4;
constexpr size_t NA_PML = (size_t)MAXT * MAXM * NQ * 4;
constexpr size_t NA_BYTES = 2 * NA_KV + NA_PO + 2 * NA_PML;  // 5,259,264
static __device__ __align__(256) uint8_t scratch[NA_BYTES];
constexpr int NA_MAXDEV = 64;
static std::mutex na_mu;
static uint8_t* na_scratch[NA_MAXDEV];

// with `device` current: the device address of its scratch (taken once)
static hipError_t na_scratch_init(int device) {
  if (device < 0 || device >= NA_MAXDEV) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(na_mu);
  if (na_scratch[device]) return hipSuccess;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  na_scratch[device] = static_cast<uint8_t*>(p);
  return hipSuccess;
}

int g4v_create(int device, g4v_ctx** out) {
  if (!out) return G4V_E_ARG;
  auto* c = new g4v_ctx();
  c->device = device;
  *out = nullptr;
  hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) {
    delete c;
    return G4V_E_HIP;
  }
  if (const char* cfg = std::getenv("G4V_GEMV_CFG")) {
    int v[8];
    if (std::sscanf(cfg, "%d,%d %d,%d %d,%d %d,%d", &v[0], &v[1], &v[2], &v[3], &v[4], &v[5], &v[6], &v[7]) == 8)
      for (int i = 0; i < 4; ++i) {
        c->gcfg[i][0] = std::min(4, std::max(1, v[2 * i]));
        c->gcfg[i][1] = v[2 * i + 1] == 32 ? 32 : 64;
      }
  }
  e = hipStreamCreate(&c->st);
  if (e != hipSuccess) {
    delete c;
    return G4V_E_HIP;
  }
  if (na_scratch_init(device) != hipSuccess) {
    delete c;
    return G4V_E_HIP;
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) == hipSuccess) {
    c->cus = prop.multiProcessorCount;
    c->lds_max = (int)std::min<size_t>(std::max<size_t>(prop.sharedMemPerBlock, prop.sharedMemPerBlockOptin), 163840);
  }
  if (hipHostMalloc((void**)&c->step_host, sizeof(StepDev)) != hipSuccess ||
      hipHostMalloc((void**)&c->res_host, sizeof(VerifyResultDev)) != hipSuccess) {
    delete c;
    return G4V_E_NOMEM;
  }
  *out = c;
  return 0;
}

void g4v_destroy(g4v_ctx* c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->st);
  delete c;
}

const char* g4v_error(const g4v_ctx* c) { return c ? c->err.c_str() : "null context"; }

int g4v_device_info(g4v_ctx* c, char* name, int cap, int* cus, int* lds) {
  hipDeviceProp_t prop;
  HIPCHK(hipGetDeviceProperties(&prop, c->device));
  if (name && cap > 0) {
    std::snprintf(name, cap, "%s (%s)", prop.name, prop.gcnArchName);
  }
  if (cus) *cus = prop.multiProcessorCount;
  if (lds) *lds = (int)prop.sharedMemPerBlock;
  return 0;
}

// ---------------------------------------------------------------------------------------
// W4G32
// ---------------------------------------------------------------------------------------
// the gate / up pair tiles of a layer, once both matrices are present
static int tile_gateup(g4v_ctx* c, Layer& L) {
  Mat& g = L.m[4];
  const Mat& u = L.m[5];
  if (!g.wr.p || !u.wr.p || g.N != u.N || g.K != u.K) return 0;
  ALLOC(g.tw, (size_t)2 * g.N * g.K / 2);
  ALLOC(g.ts, (size_t)2 * g.N * g.K / 16);
  launch_tile_w4_pair(g.wr.as<uint4>(), g.s.as<uint16_t>(), u.wr.as<uint4>(), u.s.as<uint16_t>(), g.tw.as<uint4>(),
                      g.ts.as<uint4>(), g.N, g.K, c->st);
  return 0;
}

static int upload_w4(g4v_ctx* c, Mat& m, const uint8_t* w_dev_orig, const uint16_t* s_host_or_dev, bool s_on_dev,
                     int N, int K, bool tiled = false) {
  m.N = N;
  m.K = K;
  ALLOC(m.wr, (size_t)N * K / 2);
  ALLOC(m.s, (size_t)N * K / 16);
  launch_relayout_w4(w_dev_orig, m.wr.as<uint4>(), N, K, c->st);
  HIPCHK(hipMemcpyAsync(m.s.p, s_host_or_dev, (size_t)N * K / 16,
                        s_on_dev ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, c->st));
  if (N % 16 == 0) {  // operand tiles of the W4A8 path (prefill, g4v_w4a8_gemm)
    ALLOC(m.a8w, (size_t)N * K / 2);
    ALLOC(m.a8s, (size_t)N * K / 16);
    launch_tile_a8(w_dev_orig, m.s.as<uint16_t>(), m.a8w.as<uint4>(), m.a8s.as<uint4>(), N, K, c->st);
  }
  if (tiled) {
    ALLOC(m.tw, (size_t)N * K / 2);
    ALLOC(m.ts, (size_t)N * K / 16);
    launch_tile_w4(m.wr.as<uint4>(), m.s.as<uint16_t>(), m.tw.as<uint4>(), m.ts.as<uint4>(), N, K, c->st);
  }
  return 0;
}

int g4v_w4_upload(g4v_ctx* c, const uint8_t* w, const uint16_t* s, int N, int K) {
  if (!c) return G4V_E_ARG;
  ARGCHK(w && s && N > 0 && K > 0 && K % 256 == 0, "w4_upload: need N > 0 and K % 256 == 0");
  HIPCHK(hipSetDevice(c->device));
  DBuf tmp;
  ALLOC(tmp, (size_t)N * K / 2);
  HIPCHK(hipMemcpyAsync(tmp.p, w, (size_t)N * K / 2, hipMemcpyHostToDevice, c->st));
  auto m = std::make_unique<Mat>();
  int r = upload_w4(c, *m, tmp.as<uint8_t>(), s, false, N, K);
  if (r) return r;
  HIPCHK(hipStreamSynchronize(c->st));
  c->mats.push_back(std::move(m));
  return (int)c->mats.size() - 1;
}

static int gemv_io(g4v_ctx* c, int h, int M) {
  const Mat& m = *c->mats[h];
  if (c->gx.n < (size_t)M * m.K * 4) ALLOC(c->gx, (size_t)MAXM * m.K * 4);
  if (c->gy.n < (size_t)M * m.N * 4) ALLOC(c->gy, (size_t)MAXM * m.N * 4);
  return 0;
}

static GemvArgs plain_args(const Mat& m, const float* x, float* y, int M) {
  GemvArgs a{};
  a.mat[0] = m.dev();
  a.y[0] = y;
  a.ldy[0] = m.N;
  a.x = x;
  a.ldx = m.K;
  a.K = m.K;
  a.M = M;
  return a;
}

int g4v_w4g32_gemm(g4v_ctx* c, int h, const float* x, int M, float* y) {
  if (!c) return G4V_E_ARG;
  ARGCHK(h >= 0 && h < (int)c->mats.size(), "w4g32_gemm: bad handle");
  ARGCHK(x && y && M >= 1 && M <= MAXM, "w4g32_gemm: need 1 <= M <= 8");
  HIPCHK(hipSetDevice(c->device));
  int r = gemv_io(c, h, M);
  if (r) return r;
  const Mat& m = *c->mats[h];
  HIPCHK(hipMemcpyAsync(c->gx.p, x, (size_t)M * m.K * 4, hipMemcpyHostToDevice, c->st));
  gemv_passes(c, plain_args(m, c->gx.as<float>(), c->gy.as<float>(), M), EPI_STORE, M);
  HIPCHK(hipGetLastError());
  HIPCHK(hipMemcpyAsync(y, c->gy.p, (size_t)M * m.N * 4, hipMemcpyDeviceToHost, c->st));
  HIPCHK(hipStreamSynchronize(c->st));
  return 0;
}

int g4v_w4g32_gemm_multi(g4v_ctx* c, int nmat, const int* h, const float* x, int M, float* const* y) {
  if (!c) return G4V_E_ARG;
  ARGCHK(nmat >= 1 && nmat <= 3 && h && x && y && M >= 1 && M <= MAXM, "w4g32_gemm_multi: 1 to 3 matrices, 1 <= M <= 8");
  size_t ntot = 0;
  for (int j = 0; j < nmat; ++j) {
    ARGCHK(h[j] >= 0 && h[j] < (int)c->mats.size() && y[j], "w4g32_gemm_multi: bad handle or output");
    ARGCHK(c->mats[h[j]]->K == c->mats[h[0]]->K, "w4g32_gemm_multi: the matrices need the same K");
    ntot += c->mats[h[j]]->N;
  }
  HIPCHK(hipSetDevice(c->device));
  const int K = c->mats[h[0]]->K;
  if (c->gx.n < (size_t)MAXM * K * 4) ALLOC(c->gx, (size_t)MAXM * K * 4);
  if (c->gy.n < (size_t)M * ntot * 4) ALLOC(c->gy, (size_t)MAXM * ntot * 4);
  HIPCHK(hipMemcpyAsync(c->gx.p, x, (size_t)M * K * 4, hipMemcpyHostToDevice, c->st));
  GemvArgs a{};
  size_t off = 0;
  for (int j = 0; j < nmat; ++j) {  // matrix j's rows [M][N_j] after those of the matrices before it
    const Mat& m = *c->mats[h[j]];
    a.mat[j] = m.dev();
    a.y[j] = c->gy.as<float>() + off;
    a.ldy[j] = m.N;
    off += (size_t)M * m.N;
  }
  a.x = c->gx.as<float>();
  a.ldx = K;
  a.K = K;
  gemv_passes(c, a, EPI_STORE, M);
  HIPCHK(hipGetLastError());
  off = 0;
  for (int j = 0; j < nmat; ++j) {
    const size_t n = (size_t)M * c->mats[h[j]]->N;
    HIPCHK(hipMemcpyAsync(y[j], c->gy.as<float>() + off, n * 4, hipMemcpyDeviceToHost, c->st));
    off += n;
  }
  HIPCHK(hipStreamSynchronize(c->st));
  return 0;
}

int g4v_w4g32_bench(g4v_ctx* c, int h, int M, int iters, float* us) {
  if (!c) return G4V_E_ARG;
  ARGCHK(h >= 0 && h < (int)c->mats.size() && M >= 1 && M <= MAXM && iters > 0 && us, "w4g32_bench: bad args");
  HIPCHK(hipSetDevice(c->device));
  int r = gemv_io(c, h, M);
  if (r) return r;
  const Mat& m = *c->mats[h];
  GemvArgs a = plain_args(m, c->gx.as<float>(), c->gy.as<float>(), M);
  gemv_passes(c, a, EPI_STORE, M);
  hipEvent_t e0, e1;
  HIPCHK(hipEventCreate(&e0));
  HIPCHK(hipEventCreate(&e1));
  HIPCHK(hipEventRecord(e0, c->st));
  for (int i = 0; i < iters; ++i) gemv_passes(c, a, EPI_STORE, M);
  HIPCHK(hipEventRecord(e1, c->st));
  HIPCHK(hipEventSynchronize(e1));
  float ms = 0;
  HIPCHK(hipEventElapsedTime(&ms, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  *us = ms * 1000.f / iters;
  return 0;
}

int g4v_w4g32_norm_gemm(g4v_ctx* c, int h, int mode, const float* o, const float* xin, const float* w1,
                        const float* w2, float scalar, int M, int rows_per_block, int tile_rows, float* y, float* x1) {
  if (!c) return G4V_E_ARG;
  ARGCHK(h >= 0 && h < (int)c->mats.size(), "w4g32_norm_gemm: bad handle");
  ARGCHK(mode == 1 || mode == 2, "w4g32_norm_gemm: mode 1 (after attention) or 2 (after the MLP)");
  ARGCHK(o && xin && w1 && w2 && y && x1 && M >= 1 && M <= MAXM, "w4g32_norm_gemm: need 1 <= M <= 8");
  ARGCHK(rows_per_block >= 1 && rows_per_block <= 4 && (tile_rows == 32 || tile_rows == 64),
         "w4g32_norm_gemm: 1 <= rows_per_block <= 4, tile_rows 32 or 64");
  Mat& m = *c->mats[h];
  ARGCHK(m.K == H && m.N % 64 == 0, "w4g32_norm_gemm: the matrix needs K = 1536 and N % 64 == 0");
  HIPCHK(hipSetDevice(c->device));
  if (!m.tw.p) {  // the row-tiled copy, once per handle
    ALLOC(m.tw, (size_t)m.N * m.K / 2);
    ALLOC(m.ts, (size_t)m.N * m.K / 16);
    launch_tile_w4(m.wr.as<uint4>(), m.s.as<uint16_t>(), m.tw.as<uint4>(), m.ts.as<uint4>(), m.N, m.K, c->st);
  }
  int r = gemv_io(c, h, M);
  if (r) return r;
  if (!c->nrmio.p) ALLOC(c->nrmio, ((size_t)3 * MAXM * H + 2 * H) * 4);
  float* od = c->nrmio.as<float>();
  float *xd = od + MAXM * H, *x1d = xd + MAXM * H, *w1d = x1d + MAXM * H, *w2d = w1d + H;
  HIPCHK(hipMemcpyAsync(od, o, (size_t)M * H * 4, hipMemcpyHostToDevice, c->st));
  HIPCHK(hipMemcpyAsync(xd, xin, (size_t)M * H * 4, hipMemcpyHostToDevice, c->st));
  HIPCHK(hipMemcpyAsync(w1d, w1, (size_t)H * 4, hipMemcpyHostToDevice, c->st));
  HIPCHK(hipMemcpyAsync(w2d, w2, (size_t)H * 4, hipMemcpyHostToDevice, c->st));
  GemvTArgs a{};
  a.mat[0] = m.tile();
  a.y[0] = c->gy.as<float>();
  a.ldy[0] = m.N;
  a.K = H;
  a.M = M;
  a.nrm_mode = mode;
  a.nrm_o = od;
  a.nrm_xin = xd;
  a.nrm_xout = x1d;
  a.nrm_w1 = w1d;
  a.nrm_w2 = w2d;
  a.nrm_scalar = scalar;
  launch_gemv_t(a, c->st, rows_per_block, tile_rows);
  HIPCHK(hipGetLastError());
  HIPCHK(hipMemcpyAsync(y, c->gy.p, (size_t)M * m.N * 4, hipMemcpyDeviceToHost, c->st));
  HIPCHK(hipMemcpyAsync(x1, x1d, (size_t)M * H * 4, hipMemcpyDeviceToHost, c->st));
  HIPCHK(hipStreamSynchronize(c->st));
  return 0;
}

// ---------------------------------------------------------------------------------------
// W4A8 (engine/w4a8_avx2.h, i8_task E:303-309)
// ---------------------------------------------------------------------------------------
constexpr int A8_MAXM = 8192;

// device copies of x [M][K] and the quantised operands for M rows
static int a8_io(g4v_ctx* c, int M, int K, int N) {
  const int Mpad = w4a8_mpad(M), G = K / 32;
  auto need = [&](DBuf& b, size_t n) -> int {
    if (b.n < n) return dalloc(c, b, n);
    return 0;
  };
  int r;
  if ((r = need(c->a8x, (size_t)M * K * 4)) || (r = need(c->a8xq, (size_t)Mpad * K * 2)) ||
      (r = need(c->a8sx, (size_t)G * Mpad * 4)) || (r = need(c->a8corr, (size_t)G * Mpad * 4)) ||
      (N > 0 && (r = need(c->a8y, (size_t)M * N * 4))))
    return r;
  return 0;
}

int g4v_w4a8_quant(g4v_ctx* c, const float* x, int M, int K, int8_t* q, float* sx, int32_t* sum) {
  if (!c) return G4V_E_ARG;
  ARGCHK(x && q && sx && sum && M >= 1 && M <= A8_MAXM && K > 0 && K % 256 == 0,
         "w4a8_quant: need 1 <= M <= 8192 and K % 256 == 0");
  HIPCHK(hipSetDevice(c->device));
  int r = a8_io(c, M, K, 0);
  if (r) return r;
  const int G = K / 32;
  if (c->a8q.n < (size_t)M * K) ALLOC(c->a8q, (size_t)M * K);
  if (c->a8qs.n < (size_t)M * G * 4) ALLOC(c->a8qs, (size_t)M * G * 4);
  if (c->a8qsum.n < (size_t)M * G * 4) ALLOC(c->a8qsum, (size_t)M * G * 4);
  HIPCHK(hipMemcpyAsync(c->a8x.p, x, (size_t)M * K * 4, hipMemcpyHostToDevice, c->st));
  launch_w4a8_quant(c->a8x.as<float>(), M, w4a8_mpad(M), K, c->a8xq.as<uint16_t>(), c->a8sx.as<float>(),
                    c->a8corr.as<float>(), c->a8q.as<int8_t>(), c->a8qs.as<float>(), c->a8qsum.as<int32_t>(), c->st);
  HIPCHK(hipGetLastError());
  HIPCHK(hipMemcpyAsync(q, c->a8q.p, (size_t)M * K, hipMemcpyDeviceToHost, c->st));
  HIPCHK(hipMemcpyAsync(sx, c->a8qs.p, (size_t)M * G * 4, hipMemcpyDeviceToHost, c->st));
  HIPCHK(hipMemcpyAsync(sum, c->a8qsum.p, (size_t)M * G * 4, hipMemcpyDeviceToHost, c->st));
  HIPCHK(hipStreamSynchronize(c->st));
  return 0;
}

static void a8_enqueue(g4v_ctx* c, const Mat& m, int M) {
  launch_w4a8_quant(c->a8x.as<float>(), M, w4a8_mpad(M), m.K, c->a8xq.as<uint16_t>(), c->a8sx.as<float>(),
                    c->a8corr.as<float>(), nullptr, nullptr, nullptr, c->st);
  launch_w4a8_gemm(m.a8w.as<uint4>(), m.a8s.as<uint4>(), c->a8xq.as<uint16_t>(), c->a8sx.as<float>(),
                   c->a8corr.as<float>(), c->a8y.as<float>(), M, m.N, m.K, m.N, c->st);
}

int g4v_w4a8_gemm(g4v_ctx* c, int h, const float* x, int M, float* y) {
  if (!c) return G4V_E_ARG;
  ARGCHK(h >= 0 && h < (int)c->mats.size(), "w4a8_gemm: bad handle");
  ARGCHK(x && y && M >= 1 && M <= A8_MAXM, "w4a8_gemm: need 1 <= M <= 8192");
  const Mat& m = *c->mats[h];
  ARGCHK(m.a8w.p != nullptr, "w4a8_gemm: the matrix needs N % 16 == 0");
  HIPCHK(hipSetDevice(c->device));
  int r = a8_io(c, M, m.K, m.N);
  if (r) return r;
  HIPCHK(hipMemcpyAsync(c->a8x.p, x, (size_t)M * m.K * 4, hipMemcpyHostToDevice, c->st));
  a8_enqueue(c, m, M);
  HIPCHK(hipGetLastError());
  HIPCHK(hipMemcpyAsync(y, c->a8y.p, (size_t)M * m.N * 4, hipMemcpyDeviceToHost, c->st));
  HIPCHK(hipStreamSynchronize(c->st));
  return 0;
}

int g4v_w4a8_bench(g4v_ctx* c, int h, int M, int iters, float* us) {
  if (!c) return G4V_E_ARG;
  ARGCHK(h >= 0 && h < (int)c->mats.size() && M >= 1 && M <= A8_MAXM && iters > 0 && us, "w4a8_bench: bad args");
  const Mat& m = *c->mats[h];
  ARGCHK(m.a8w.p != nullptr, "w4a8_bench: the matrix needs N % 16 == 0");
  HIPCHK(hipSetDevice(c->device));
  int r = a8_io(c, M, m.K, m.N);
  if (r) return r;
  HIPCHK(hipMemsetAsync(c->a8x.p, 0, (size_t)M * m.K * 4, c->st));
  a8_enqueue(c, m, M);
  hipEvent_t e0, e1;
  HIPCHK(hipEventCreate(&e0));
  HIPCHK(hipEventCreate(&e1));
  HIPCHK(hipEventRecord(e0, c->st));
  for (int i = 0; i < iters; ++i) a8_enqueue(c, m, M);
  HIPCHK(hipEventRecord(e1, c->st));
  HIPCHK(hipEventSynchronize(e1));
  float ms = 0;
  HIPCHK(hipEventElapsedTime(&ms, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  *us = ms * 1000.f / iters;
  return 0;
}

// ---------------------------------------------------------------------------------------
// attention
// ---------------------------------------------------------------------------------------
// head dim 512 (the global layers of the Gemma-4-E2B layout): g4v_attn_hd.hip
static int attn_splitkv_512(g4v_ctx* c, const uint16_t* Kc, const uint16_t* Vc, int npos, int M, const float* q,
                            const int* pos, const int* lo, const int* skip_lo, const int* skip_hi, int kmin, int kmax,
                            int nsplit, float* out) {
  constexpr int D = 512;
  AttnGeom g{};
  g.M = M;
  g.kmin = kmin;
  g.kmax = kmax;
  g.T = nsplit;
  for (int m = 0; m < M; ++m) {
    ARGCHK(pos[m] < npos, "attn_splitkv: pos beyond npos");
    g.pos[m] = pos[m];
    g.lo[m] = lo[m];
    g.skip_lo[m] = skip_lo[m];
    g.skip_hi[m] = skip_hi[m];
  }
  HIPCHK(hipSetDevice(c->device));
  const size_t kvb = (size_t)kv_cap(npos) * D * 2;
  if (c->ak.n < kvb) ALLOC(c->ak, kvb);
  if (c->av.n < kvb) ALLOC(c->av, kvb);
  if (c->aq.n < (size_t)MAXM * NQ * D * 4) ALLOC(c->aq, (size_t)MAXM * NQ * D * 4);
  if (c->ao.n < (size_t)MAXM * NQ * D * 4) ALLOC(c->ao, (size_t)MAXM * NQ * D * 4);
  if (c->po5.n < (size_t)MAXT * MAXM * NQ * D * 4) {
    ALLOC(c->po5, (size_t)MAXT * MAXM * NQ * D * 4);
    ALLOC(c->pm5, (size_t)MAXT * MAXM * NQ * 4);
    ALLOC(c->pl5, (size_t)MAXT * MAXM * NQ * 4);
  }
  {  // the caller's [position][512] rows into the device cache layout
    std::vector<uint16_t> kd((size_t)kv_cap(npos) * D, 0), vd((size_t)kv_cap(npos) * D, 0);
    for (int p = 0; p < npos; ++p)
      for (int e = 0; e < D; ++e) {
        kd[kc_index_d<D>(p, e)] = Kc[(size_t)p * D + e];
        vd[vc_index_d<D>(p, e)] = Vc[(size_t)p * D + e];
      }
    HIPCHK(hipMemcpy(c->ak.p, kd.data(), kvb, hipMemcpyHostToDevice));
    HIPCHK(hipMemcpy(c->av.p, vd.data(), kvb, hipMemcpyHostToDevice));
  }
  HIPCHK(hipMemcpyAsync(c->aq.p, q, (size_t)M * NQ * D * 4, hipMemcpyHostToDevice, c->st));
  ARGCHK(launch_attn_geom_hd(c->ak.as<uint16_t>(), c->av.as<uint16_t>(), c->aq.as<float>(), NQ * D, g, D,
                             c->po5.as<float>(), c->pm5.as<float>(), c->pl5.as<float>(), c->ao.as<float>(), NQ * D,
                             nullptr, c->st) == 0,
         "attn_splitkv: shape not served at head dim 512");
  HIPCHK(hipGetLastError());
  HIPCHK(hipMemcpyAsync(out, c->ao.p, (size_t)M * NQ * D * 4, hipMemcpyDeviceToHost, c->st));
  HIPCHK(hipStreamSynchronize(c->st));
  return 0;
}

int g4v_attn_splitkv(g4v_ctx* c, const uint16_t* Kc, const uint16_t* Vc, int npos, int hd, int nh, int M,
                     const float* q, const int* pos, const int* lo, const int* skip_lo, const int* skip_hi,
                     int kmin, int kmax, int nsplit, float* out) {
  if (!c) return G4V_E_ARG;
  ARGCHK((hd == HD || hd == 512) && nh == NQ, "attn_splitkv: hd must be 256 or 512 and nh 8");
  ARGCHK(M >= 1 && M <= MAXM && nsplit >= 1 && nsplit <= MAXT, "attn_splitkv: 1 <= M <= 8, 1 <= nsplit <= 16");
  ARGCHK(kmin >= 0 && kmax < npos && kmin <= kmax, "attn_splitkv: need 0 <= kmin <= kmax < npos");
  const int len = kmax - kmin + 1, per = (len + nsplit - 1) / nsplit;
  ARGCHK(per <= (hd == HD ? attn_pmax() : ATT_SPLIT_MAX - 1),
         "attn_splitkv: more positions per split than the split buffer holds");
  if (hd == 512) return attn_splitkv_512(c, Kc, Vc, npos, M, q, pos, lo, skip_lo, skip_hi, kmin, kmax, nsplit, out);
  AttnGeom g{};
  g.M = M;
  g.kmin = kmin;
  g.kmax = kmax;
  g.T = nsplit;
  for (int m = 0; m < M; ++m) {
    ARGCHK(pos[m] < npos, "attn_splitkv: pos beyond npos");
    g.pos[m] = pos[m];
    g.lo[m] = lo[m];
    g.skip_lo[m] = skip_lo[m];
    g.skip_hi[m] = skip_hi[m];
  }
  HIPCHK(hipSetDevice(c->device));
  const size_t kvb = (size_t)kv_cap(npos) * HD * 2;
  if (c->ak.n < kvb) ALLOC(c->ak, kvb);
  if (c->av.n < kvb) ALLOC(c->av, kvb);
  if (c->aq.n < (size_t)MAXM * NQ * HD * 4) ALLOC(c->aq, (size_t)MAXM * NQ * HD * 4);
  if (c->ao.n < (size_t)MAXM * NQ * HD * 4) ALLOC(c->ao, (size_t)MAXM * NQ * HD * 4);
  if (c->po.n < (size_t)MAXT * MAXM * NQ * HD * 4) {
    drop_graphs(c);  // the split partials are shared with the captured verify steps
    ALLOC(c->po, (size_t)MAXT * MAXM * NQ * HD * 4);
    ALLOC(c->pm, (size_t)MAXT * MAXM * NQ * 4);
    ALLOC(c->pl, (size_t)MAXT * MAXM * NQ * 4);
  }
  {  // the caller's [position][256] rows into the device cache layout
    std::vector<uint16_t> kd((size_t)kv_cap(npos) * HD, 0), vd((size_t)kv_cap(npos) * HD, 0);
    for (int p = 0; p < npos; ++p)
      for (int e = 0; e < HD; ++e) {
        kd[kc_index(p, e)] = Kc[(size_t)p * HD + e];
        vd[vc_index(p, e)] = Vc[(size_t)p * HD + e];
      }
    HIPCHK(hipMemcpy(c->ak.p, kd.data(), kvb, hipMemcpyHostToDevice));
    HIPCHK(hipMemcpy(c->av.p, vd.data(), kvb, hipMemcpyHostToDevice));
  }
  HIPCHK(hipMemcpyAsync(c->aq.p, q, (size_t)M * NQ * HD * 4, hipMemcpyHostToDevice, c->st));
  launch_attn_geom(c->ak.as<uint16_t>(), c->av.as<uint16_t>(), c->aq.as<float>(), NQ * HD, g, c->po.as<float>(),
                   c->pm.as<float>(), c->pl.as<float>(), c->ao.as<float>(), NQ * HD, c->st);
  HIPCHK(hipGetLastError());
  HIPCHK(hipMemcpyAsync(out, c->ao.p, (size_t)M * NQ * HD * 4, hipMemcpyDeviceToHost, c->st));
  HIPCHK(hipStreamSynchronize(c->st));
  return 0;
}

// the same split-KV attention on device buffers, allocating nothing: the relaid key / value rows
// and the split partials live in the file-scope scratch (NA_NPOS positions at most)
int g4v_attn_splitkv_noalloc(g4v_ctx* c, const uint16_t* Kc, const uint16_t* Vc, int npos, int hd, int nh, int M,
                             const float* q, const int* pos, const int* lo, const int* skip_lo, const int* skip_hi,
                             int kmin, int kmax, int nsplit, float* out) {
  if (!c) return G4V_E_ARG;
  ARGCHK(Kc && Vc && q && out && pos && lo && skip_lo && skip_hi, "attn_splitkv_noalloc: null pointer");
  ARGCHK(hd == HD && nh == NQ, "attn_splitkv_noalloc: hd must be 256 and nh 8");
  ARGCHK(M >= 1 && M <= MAXM && nsplit >= 1 && nsplit <= MAXT,
         "attn_splitkv_noalloc: 1 <= M <= 8, 1 <= nsplit <= 16");
  ARGCHK(npos >= 1 && npos <= NA_NPOS, "attn_splitkv_noalloc: npos beyond the scratch's 4096 positions");
  ARGCHK(kmin >= 0 && kmax < npos && kmin <= kmax, "attn_splitkv_noalloc: need 0 <= kmin <= kmax < npos");
  const int len = kmax - kmin + 1, per = (len + nsplit - 1) / nsplit;
  ARGCHK(per <= attn_pmax(), "attn_splitkv_noalloc: more positions per split than the split buffer holds");
  AttnGeom g{};
  g.M = M;
  g.kmin = kmin;
  g.kmax = kmax;
  g.T = nsplit;
  for (int m = 0; m < M; ++m) {
    ARGCHK(pos[m] >= 0 && pos[m] < npos, "attn_splitkv_noalloc: pos beyond npos");
    g.pos[m] = pos[m];
    g.lo[m] = lo[m];
    g.skip_lo[m] = skip_lo[m];
    g.skip_hi[m] = skip_hi[m];
  }
  HIPCHK(hipSetDevice(c->device));
  uint8_t* sc = c->device < NA_MAXDEV ? na_scratch[c->device] : nullptr;
  ARGCHK(sc != nullptr, "attn_splitkv_noalloc: no scratch on this device");
  uint16_t* kd = reinterpret_cast<uint16_t*>(sc);
  uint16_t* vd = reinterpret_cast<uint16_t*>(sc + NA_KV);
  float* po = reinterpret_cast<float*>(sc + 2 * NA_KV);
  float* pm = reinterpret_cast<float*>(sc + 2 * NA_KV + NA_PO);
  float* pl = reinterpret_cast<float*>(sc + 2 * NA_KV + NA_PO + NA_PML);
  launch_kv_to_cache(Kc, Vc, npos, kd, vd, c->st);
  launch_attn_geom(kd, vd, q, NQ * HD, g, po, pm, pl, out, NQ * HD, c->st);
  HIPCHK(hipGetLastError());
  HIPCHK(hipStreamSynchronize(c->st));
  return 0;
}

// ---------------------------------------------------------------------------------------
// head
// ---------------------------------------------------------------------------------------
// one head pass scores up to MAXM rows (a chain of 7 drafts evaluates 7 rows in its second pass)
static int alloc_head_bufs(g4v_ctx* c, HeadBufs& b, int V) {
  ALLOC(b.u, (size_t)MAXM * V * 4);
  ALLOC(b.list, (size_t)MAXM * HEAD_LIMIT * 4);
  ALLOC(b.sval, (size_t)MAXM * HEAD_LIMIT * 4);
  ALLOC(b.small, 5 * MAXM * 4);
  ALLOC(b.part, (size_t)2 * MAXM * HEAD_MAXGRID * 4);
  int* s = b.small.as<int>();
  b.hs.u = b.u.as<float>();
  b.hs.list = b.list.as<int>();
  b.hs.sval = b.sval.as<float>();
  b.hs.cnt = s;
  b.hs.lmax_key = s + MAXM;
  b.hs.vmax_key = s + 2 * MAXM;
  b.hs.best = s + 3 * MAXM;
  b.hs.thr = reinterpret_cast<float*>(s + 4 * MAXM);
  b.hs.lpart = b.part.as<float>();
  b.hs.vpart = b.part.as<float>() + (size_t)MAXM * HEAD_MAXGRID;
  return 0;
}

// build the screen, exp3 (dec16 + exceptions) and cap table from c->E (device, [V][H] bf16)
static int head_build_dev(g4v_ctx* c, int V) {
  drop_graphs(c);
  c->V = V;
  hipStream_t st = c->st;
  DBuf hist, gcnt, rowcnt;
  ALLOC(hist, 256 * 8);
  HIPCHK(hipMemsetAsync(hist.p, 0, 256 * 8, st));
  HeadBuildTmp tmp{hist.as<unsigned long long>(), nullptr, nullptr};
  head_build(c->E.as<uint16_t>(), V, c->hd, tmp, st);
  std::vector<unsigned long long> hh(256);
  HIPCHK(hipMemcpyAsync(hh.data(), hist.p, 256 * 8, hipMemcpyDeviceToHost, st));
  HIPCHK(hipStreamSynchronize(st));
  // E:1232-1234: the 8 most frequent exponents, stable order
  std::vector<int> ord(256);
  for (int i = 0; i < 256; ++i) ord[i] = i;
  std::stable_sort(ord.begin(), ord.end(), [&](int a, int b) { return hh[a] > hh[b]; });
  uint8_t cb8[8];
  for (int i = 0; i < 8; ++i) cb8[i] = (uint8_t)ord[i];
  ALLOC(c->cb, 16);
  HIPCHK(hipMemcpyAsync(c->cb.p, cb8, 8, hipMemcpyHostToDevice, st));
  ALLOC(c->dec, (size_t)V * H * 2);
  ALLOC(gcnt, (size_t)V * 48);
  ALLOC(rowcnt, (size_t)V * 4);
  c->hd = HeadDev{};
  c->hd.dec = c->dec.as<uint4>();
  c->hd.decw = c->dec.as<uint4>();
  c->hd.cb = c->cb.as<uint8_t>();
  tmp.gcnt = gcnt.as<uint8_t>();
  tmp.rowcnt = rowcnt.as<int>();
  head_build_dec(c->E.as<uint16_t>(), V, c->hd, tmp, st);
  std::vector<int> rc(V), ptr(V + 1);
  HIPCHK(hipMemcpyAsync(rc.data(), rowcnt.p, (size_t)V * 4, hipMemcpyDeviceToHost, st));
  HIPCHK(hipStreamSynchronize(st));
  ptr[0] = 0;
  for (int n = 0; n < V; ++n) ptr[n + 1] = ptr[n] + rc[n];
  const int ne = ptr[V];
  ALLOC(c->exc_ptr, (size_t)(V + 1) * 4);
  ALLOC(c->exc_col, (size_t)(ne + 1) * 2);
  ALLOC(c->exc_del, (size_t)(ne + 1) * 4);
  HIPCHK(hipMemcpyAsync(c->exc_ptr.p, ptr.data(), (size_t)(V + 1) * 4, hipMemcpyHostToDevice, st));
  c->hd.exc_ptr = c->exc_ptr.as<int>();
  c->hd.exc_col = c->exc_col.as<uint16_t>();
  c->hd.exc_del = c->exc_del.as<float>();
  c->hd.exc_col_w = c->exc_col.as<uint16_t>();
  c->hd.exc_del_w = c->exc_del.as<float>();
  head_build_exc(c->E.as<uint16_t>(), V, c->hd, st);
  ALLOC(c->x3sm, (size_t)V * 24 * 8 * 8);
  ALLOC(c->x3ix, (size_t)V * 24 * 8 * 4);
  c->hd.x3sm = c->x3sm.as<uint2>();
  c->hd.x3ix = c->x3ix.as<uint32_t>();
  c->hd.x3smw = c->x3sm.as<uint2>();
  c->hd.x3ixw = c->x3ix.as<uint32_t>();
  head_build_x3(V, c->hd, st);
  // E:1236-1243 screen
  DBuf wq;
  ALLOC(wq, (size_t)V * H / 2);
  ALLOC(c->scr_s, (size_t)V * H / 16);
  ALLOC(c->coef, (size_t)V * 4);
  screen_build(c->E.as<uint16_t>(), V, wq.as<uint8_t>(), c->scr_s.as<uint16_t>(), c->coef.as<float>(), st);
  ALLOC(c->scr_wr, (size_t)V * H / 2);
  launch_relayout_w4(wq.as<uint8_t>(), c->scr_wr.as<uint4>(), V, H, st);
  // cap(v) = r16(30 tanhf(v / 30)) over every bf16 input, with the host libm (E:1409)
  std::vector<uint16_t> lut(65536);
  for (int b = 0; b < 65536; ++b) lut[b] = f2bf(30.0f * tanhf(bf2f((uint16_t)b) / 30.0f));
  ALLOC(c->lut, 65536 * 2);
  HIPCHK(hipMemcpyAsync(c->lut.p, lut.data(), 65536 * 2, hipMemcpyHostToDevice, st));
  int r = alloc_head_bufs(c, c->hb1, V);
  if (r) return r;
  r = alloc_head_bufs(c, c->hb2, V);
  if (r) return r;
  ALLOC(c->hrow, (size_t)4 * H * 4);
  ALLOC(c->hnrow, 4 * 4);
  HIPCHK(hipGetLastError());
  HIPCHK(hipStreamSynchronize(st));
  c->head_ready = true;
  return 0;
}

int g4v_head_build(g4v_ctx* c, const uint16_t* E, int V) {
  if (!c) return G4V_E_ARG;
  ARGCHK(E && V > 0, "head_build: need E and V > 0");
  HIPCHK(hipSetDevice(c->device));
  drop_graphs(c);  // E and the head buffers are reallocated
  ALLOC(c->E, (size_t)V * H * 2);
  HIPCHK(hipMemcpyAsync(c->E.p, E, (size_t)V * H * 2, hipMemcpyHostToDevice, c->st));
  return head_build_dev(c, V);
}

static HeadRun head_args(g4v_ctx* c, HeadBufs& b, const float* h, const float* hn, int MT, const int* active) {
  HeadRun r{};
  r.prof.mark = pmark;
  r.prof.ctx = c;
  // one full-head pass reads every decoded row (V x 1536 bf16), the row pointers and the exceptions
  r.full_bytes = (double)c->V * 24 * 8 * 12 + (double)(c->V + 1) * 4 + (double)c->exc_col.n / 2 * 6;
  r.hs = b.hs;
  r.hd = c->hd;
  r.screen = W4Dev{c->scr_wr.as<uint4>(), c->scr_s.as<uint16_t>(), c->V, H};
  r.coef = c->coef.as<float>();
  r.lut = c->lut.as<uint16_t>();
  r.h = h;
  r.hn = hn;
  r.active = active;
  r.MT = MT;
  r.V = c->V;
  r.grid_cap = (c->cus > 0 ? c->cus : 256) * 8;  // grid-stride: stage the rows once per block
  return r;
}

int g4v_head_argmax(g4v_ctx* c, const float* h, int M, int* G, int* nsurv, int* fallback) {
  if (!c) return G4V_E_ARG;
  if (!c->head_ready) {
    c->err = "head_argmax: no head (g4v_head_build or g4v_model_synth first)";
    return G4V_E_STATE;
  }
  ARGCHK(h && G && M >= 1 && M <= 4, "head_argmax: 1 <= M <= 4");
  HIPCHK(hipSetDevice(c->device));
  std::vector<float> hn(M);
  for (int m = 0; m < M; ++m) {  // E:1417 |h| = (float)sqrt(ss_avx2(h)) in the reference's order
    double s[16] = {0};
    for (int i = 0; i < H; ++i) {
      const double d = h[(size_t)m * H + i];
      s[i % 16] = std::fma(d, d, s[i % 16]);
    }
    double a[4];
    for (int l = 0; l < 4; ++l) a[l] = (s[l] + s[4 + l]) + (s[8 + l] + s[12 + l]);
    hn[m] = (float)std::sqrt((a[0] + a[2]) + (a[1] + a[3]));
  }
  HIPCHK(hipMemcpyAsync(c->hrow.p, h, (size_t)M * H * 4, hipMemcpyHostToDevice, c->st));
  HIPCHK(hipMemcpyAsync(c->hnrow.p, hn.data(), (size_t)M * 4, hipMemcpyHostToDevice, c->st));
  head_run(head_args(c, c->hb1, c->hrow.as<float>(), c->hnrow.as<float>(), M, nullptr), c->st);
  HIPCHK(hipGetLastError());
  int small[4 * MAXM];
  HIPCHK(hipMemcpyAsync(small, c->hb1.small.p, sizeof small, hipMemcpyDeviceToHost, c->st));
  HIPCHK(hipStreamSynchronize(c->st));
  for (int m = 0; m < M; ++m) {
    G[m] = small[3 * MAXM + m];
    if (nsurv) nsurv[m] = small[m];
    if (fallback) fallback[m] = small[m] > HEAD_LIMIT;
  }
  if (c->prof_mask) prof_collect(c, small[0] > HEAD_LIMIT);
  return 0;
}

int g4v_head_survivors(g4v_ctx* c, int m, int* idx, float* val, int cap, int* n) {
  if (!c) return G4V_E_ARG;
  ARGCHK(m >= 0 && m < 4 && idx && val && n, "head_survivors: bad args");
  int cnt = 0;
  HIPCHK(hipMemcpy(&cnt, c->hb1.hs.cnt + m, 4, hipMemcpyDeviceToHost));
  *n = cnt;
  if (cnt > HEAD_LIMIT) return 0;
  const int k = std::min(cnt, cap);
  std::vector<int> li(cnt);
  std::vector<float> lv(cnt);
  HIPCHK(hipMemcpy(li.data(), c->hb1.hs.list + (size_t)m * HEAD_LIMIT, (size_t)cnt * 4, hipMemcpyDeviceToHost));
  HIPCHK(hipMemcpy(lv.data(), c->hb1.hs.sval + (size_t)m * HEAD_LIMIT, (size_t)cnt * 4, hipMemcpyDeviceToHost));
  std::vector<int> o(cnt);
  for (int i = 0; i < cnt; ++i) o[i] = i;
  std::sort(o.begin(), o.end(), [&](int a, int b) { return li[a] < li[b]; });
  for (int i = 0; i < k; ++i) {
    idx[i] = li[o[i]];
    val[i] = lv[o[i]];
  }
  return 0;
}

// ---------------------------------------------------------------------------------------
// synthetic model
// ---------------------------------------------------------------------------------------
}  // extern "C"

// Allocate an empty stack of NL layers: matrices unset, norms zero, KV cache zeroed, RoPE
// tables (E:1246-1248: sliding layers theta 1e4 full rotary, global layers 1e6 rotary 0.25)
// and the step buffers.  The weights come from model_synth or from the g4v_model_set_* calls.
static int model_alloc(g4v_ctx* c, int V, int NL, int I, int ctxcap) {
  hipStream_t st = c->st;
  drop_graphs(c);  // every model and step buffer is reallocated below
  c->model_ready = false;
  c->head_ready = false;
  c->gemma = false;
  c->V = V;
  c->NL = NL;
  c->I = I;
  c->ctxcap = ctxcap;
  c->kvcap = kv_cap(ctxcap);
  ALLOC(c->E, (size_t)V * H * 2);
  c->L.clear();
  for (int l = 0; l < NL; ++l) {
    auto lay = std::make_unique<Layer>();
    ALLOC(lay->norms, (size_t)(4 * H + 4 * HD) * 4);
    HIPCHK(hipMemsetAsync(lay->norms.p, 0, lay->norms.n, st));
    lay->scalar = 1.0f;
    lay->sliding = (l % 5 != 4);
    c->L.push_back(std::move(lay));
  }
  ALLOC(c->fnorm, H * 4);
  HIPCHK(hipMemsetAsync(c->fnorm.p, 0, H * 4, st));
  ALLOC(c->KC, (size_t)NL * c->kvcap * HD * 2);
  ALLOC(c->VC, (size_t)NL * c->kvcap * HD * 2);
  HIPCHK(hipMemsetAsync(c->KC.p, 0, c->KC.n, st));
  HIPCHK(hipMemsetAsync(c->VC.p, 0, c->VC.n, st));
  std::vector<float> rt((size_t)4 * ctxcap * (HD / 2));
  for (int ty = 0; ty < 2; ++ty) {
    const double theta = ty ? 1e6 : 1e4;
    const int ra = (int)(HD * (ty ? 0.25 : 1.0)) / 2;
    float* cs = rt.data() + (size_t)(2 * ty) * ctxcap * (HD / 2);
    float* sn = cs + (size_t)ctxcap * (HD / 2);
    for (int p = 0; p < ctxcap; ++p)
      for (int j = 0; j < HD / 2; ++j) {
        const double inv = j < ra ? 1.0 / std::pow(theta, (2.0 * j) / HD) : 0.0;
        const double ang = p * inv;
        cs[(size_t)p * (HD / 2) + j] = (float)std::cos(ang);
        sn[(size_t)p * (HD / 2) + j] = (float)std::sin(ang);
      }
  }
  ALLOC(c->rope, rt.size() * 4);
  ALLOC(c->ropestep, (size_t)2 * MAXM * HD * 4);
  HIPCHK(hipMemcpyAsync(c->rope.p, rt.data(), rt.size() * 4, hipMemcpyHostToDevice, st));
  ALLOC(c->x, MAXM * H * 4);
  ALLOC(c->x2, MAXM * H * 4);
  ALLOC(c->xa, MAXM * H * 4);
  ALLOC(c->xgs, MAXM * (H / 32) * 4);
  ALLOC(c->q, MAXM * NQ * HD * 4);
  ALLOC(c->k, MAXM * HD * 4);
  ALLOC(c->v, MAXM * HD * 4);
  ALLOC(c->o, MAXM * H * 4);
  ALLOC(c->act, (size_t)MAXM * I * 4);
  ALLOC(c->h, MAXM * H * 4);
  ALLOC(c->hn, MAXM * 4);
  ALLOC(c->h2, MAXM * H * 4);
  ALLOC(c->hn2, MAXM * 4);
  ALLOC(c->po, (size_t)MAXT * MAXM * NQ * HD * 4);
  ALLOC(c->pm, (size_t)MAXT * MAXM * NQ * 4);
  ALLOC(c->pl, (size_t)MAXT * MAXM * NQ * 4);
  ALLOC(c->stepd, sizeof(StepDev));
  ALLOC(c->vatt, (size_t)MAXM * NQ * HD * 4);
  ALLOC(c->vags, (size_t)MAXM * NQ * HD / 32 * 4);
  ALLOC(c->q8w, (size_t)MAXM * 384 * 32);
  ALLOC(c->q8s, (size_t)MAXM * 384 * 4);
  ALLOC(c->vsc, (size_t)8 * MAXM * ctxcap * 4);
  ALLOC(c->resd, sizeof(VerifyResultDev));
  HIPCHK(hipStreamSynchronize(st));  // rt goes out of scope
  return 0;
}

static const int kMatN[7] = {NQ * HD, HD, HD, H, 0, 0, H}, kMatK[7] = {H, H, H, NQ * HD, H, H, 0};
static int mat_n(const g4v_ctx* c, int j) { return (j == 4 || j == 5) ? c->I : kMatN[j]; }
static int mat_k(const g4v_ctx* c, int j) { return j == 6 ? c->I : kMatK[j]; }

// every matrix, the embedding/head and the norms are present
static bool model_complete(const g4v_ctx* c, std::string* what) {
  if (c->L.empty()) {
    *what = "no model";
    return false;
  }
  if (!c->head_ready) {
    *what = "embedding / head not set";
    return false;
  }
  for (int l = 0; l < (int)c->L.size(); ++l)
    for (int j = 0; j < 7; ++j)
      if (!c->L[l]->m[j].wr.p) {
        *what = "matrix " + std::to_string(j) + " of layer " + std::to_string(l) + " not set";
        return false;
      }
  return true;
}

extern "C" {

int g4v_model_synth(g4v_ctx* c, uint64_t seed, int V, int NL, int I, int ctxcap) {
  if (!c) return G4V_E_ARG;
  ARGCHK(V > 0 && NL > 0 && NL <= 64 && I > 0 && I % 256 == 0 && (I <= 6144 || I == 12288) && ctxcap > 8,
         "model_synth: need I % 256 == 0, I <= 6144 or I = 12288");
  HIPCHK(hipSetDevice(c->device));
  hipStream_t st = c->st;
  int r = model_alloc(c, V, NL, I, ctxcap);
  if (r) return r;
  // output matrix / embedding: E[n][k] = f2bf(0.02 normal(stream(seed, 1), n*H + k))
  launch_gen_bf16_normal(c->E.as<uint16_t>(), (size_t)V * H, rng_stream(seed, 1), 0.02f, st);
  r = head_build_dev(c, V);
  if (r) return r;
  c->head_ready = true;
  DBuf tw, ts;
  ALLOC(tw, (size_t)std::max(I, NQ * HD) * std::max(H, I) / 2);
  ALLOC(ts, (size_t)std::max(I, NQ * HD) * std::max(H, I) / 16);
  std::vector<float> nv(4 * H + 2 * HD);
  for (int l = 0; l < NL; ++l) {
    Layer& lay = *c->L[l];
    for (int j = 0; j < 7; ++j) {
      const int N = mat_n(c, j), K = mat_k(c, j);
      const size_t nb = (size_t)N * K / 2, ns = (size_t)N * K / 32;
      launch_gen_w4(tw.as<uint8_t>(), ts.as<uint16_t>(), nb, ns, rng_stream(seed, 1000 + 10 * (uint64_t)l + j),
                    rng_stream(seed, 2000 + 10 * (uint64_t)l + j), st);
      r = upload_w4(c, lay.m[j], tw.as<uint8_t>(), ts.as<uint16_t>(), true, N, K, row_tiled(j));
      if (r) return r;
    }
    r = tile_gateup(c, lay);
    if (r) return r;
    // norms: r16(base + span * unif(stream(seed, 3000 + 10 l + t), i))
    for (int t = 0; t < 6; ++t) {
      const int n = t < 4 ? H : HD, off = t < 4 ? t * H : 4 * H + (t - 4) * HD;
      const float base = t < 4 ? 0.5f : 0.2f, span = t < 4 ? 1.0f : 0.1f;
      const uint64_t sn = rng_stream(seed, 3000 + 10 * (uint64_t)l + t);
      for (int i = 0; i < n; ++i) nv[off + i] = r16(base + span * rng_unif(sn, i));
    }
    HIPCHK(hipMemcpyAsync(lay.norms.p, nv.data(), nv.size() * 4, hipMemcpyHostToDevice, st));
    lay.perm_norms(st);
    HIPCHK(hipStreamSynchronize(st));  // nv is refilled for the next layer
    lay.scalar = 0.75f;
    lay.sliding = (l % 5 != 4);
  }
  std::vector<float> fn(H);
  const uint64_t sf = rng_stream(seed, 4000);
  for (int i = 0; i < H; ++i) fn[i] = r16(0.5f + rng_unif(sf, i));
  HIPCHK(hipMemcpyAsync(c->fnorm.p, fn.data(), H * 4, hipMemcpyHostToDevice, st));
  HIPCHK(hipGetLastError());
  HIPCHK(hipStreamSynchronize(st));
  c->model_ready = true;
  return 0;
}

int g4v_model_create(g4v_ctx* c, int V, int NL, int I, int ctxcap) {
  if (!c) return G4V_E_ARG;
  ARGCHK(V > 0 && NL > 0 && NL <= 64 && I > 0 && I % 256 == 0 && (I <= 6144 || I == 12288) && ctxcap > 8,
         "model_create: need I % 256 == 0, I <= 6144 or I = 12288");
  HIPCHK(hipSetDevice(c->device));
  int r = model_alloc(c, V, NL, I, ctxcap);
  if (r) return r;
  c->model_ready = true;
  return 0;
}

int g4v_model_set_embed(g4v_ctx* c, const uint16_t* E) {
  if (!c || !E) return G4V_E_ARG;
  if (c->L.empty()) {
    c->err = "model_set_embed: no model (g4v_model_create first)";
    return G4V_E_STATE;
  }
  HIPCHK(hipSetDevice(c->device));
  HIPCHK(hipMemcpyAsync(c->E.p, E, (size_t)c->V * H * 2, hipMemcpyHostToDevice, c->st));
  int r = head_build_dev(c, c->V);
  if (r) return r;
  HIPCHK(hipStreamSynchronize(c->st));
  c->head_ready = true;
  return 0;
}

static int gm_set_matrix(g4v_ctx* c, int l, int j, const uint8_t* w, const uint16_t* s);

int g4v_model_set_matrix(g4v_ctx* c, int l, int j, const uint8_t* w, const uint16_t* s) {
  if (!c || !w || !s) return G4V_E_ARG;
  if (c->gemma) {
    HIPCHK(hipSetDevice(c->device));
    return gm_set_matrix(c, l, j, w, s);
  }
  ARGCHK(l >= 0 && l < (int)c->L.size() && j >= 0 && j < 7, "model_set_matrix: layer or matrix index out of range");
  HIPCHK(hipSetDevice(c->device));
  drop_graphs(c);  // the matrix buffers are reallocated
  const int N = mat_n(c, j), K = mat_k(c, j);
  DBuf tmp;
  ALLOC(tmp, (size_t)N * K / 2);
  HIPCHK(hipMemcpyAsync(tmp.p, w, (size_t)N * K / 2, hipMemcpyHostToDevice, c->st));
  int r = upload_w4(c, c->L[l]->m[j], tmp.as<uint8_t>(), s, false, N, K, row_tiled(j));
  if (r) return r;
  if (j == 4 || j == 5) r = tile_gateup(c, *c->L[l]);
  if (r) return r;
  HIPCHK(hipStreamSynchronize(c->st));
  return 0;
}

int g4v_model_set_norms(g4v_ctx* c, int l, const float* const nv[6], float scalar, int sliding) {
  if (!c || !nv) return G4V_E_ARG;
  ARGCHK(l >= 0 && l < (int)c->L.size(), "model_set_norms: layer index out of range");
  for (int t = 0; t < 6; ++t) ARGCHK(nv[t] != nullptr, "model_set_norms: null norm vector");
  HIPCHK(hipSetDevice(c->device));
  Layer& lay = *c->L[l];
  for (int t = 0; t < 6; ++t) {
    const int n = t < 4 ? H : HD, off = t < 4 ? t * H : 4 * H + (t - 4) * HD;
    HIPCHK(hipMemcpyAsync(lay.norms.as<float>() + off, nv[t], (size_t)n * 4, hipMemcpyHostToDevice, c->st));
  }
  lay.perm_norms(c->st);
  HIPCHK(hipGetLastError());
  HIPCHK(hipStreamSynchronize(c->st));
  if (lay.scalar != scalar || lay.sliding != (sliding != 0)) drop_graphs(c);  // both are baked into launches
  lay.scalar = scalar;
  lay.sliding = sliding != 0;
  return 0;
}

int g4v_model_set_final_norm(g4v_ctx* c, const float* w) {
  if (!c || !w) return G4V_E_ARG;
  if (c->L.empty()) {
    c->err = "model_set_final_norm: no model";
    return G4V_E_STATE;
  }
  HIPCHK(hipSetDevice(c->device));
  HIPCHK(hipMemcpyAsync(c->fnorm.p, w, H * 4, hipMemcpyHostToDevice, c->st));
  HIPCHK(hipStreamSynchronize(c->st));
  return 0;
}

// reference rows K, V [n][256] for positions pos0 .. pos0 + n - 1 of layer l, written in the
// device cache layout (kc_index / vc_index); the value blocks they touch are read, patched and
// written back so that the block's other positions keep their contents
static int kv_upload(g4v_ctx* c, int l, int pos0, int n, const uint16_t* K, const uint16_t* V) {
  if (n <= 0) return 0;
  uint16_t* kslab = c->KC.as<uint16_t>() + (size_t)l * c->kvcap * HD;
  uint16_t* vslab = c->VC.as<uint16_t>() + (size_t)l * c->kvcap * HD;
  std::vector<uint16_t> kd((size_t)n * HD);
  for (int r = 0; r < n; ++r)
    for (int e = 0; e < HD; ++e) kd[(size_t)r * HD + kc_slot(e)] = K[(size_t)r * HD + e];
  HIPCHK(hipMemcpy(kslab + (size_t)pos0 * HD, kd.data(), kd.size() * 2, hipMemcpyHostToDevice));
  const int b0 = pos0 / 32, b1 = (pos0 + n - 1) / 32;
  std::vector<uint16_t> vd((size_t)(b1 - b0 + 1) * 32 * HD);
  uint16_t* vblk = vslab + (size_t)b0 * 32 * HD;
  HIPCHK(hipMemcpy(vd.data(), vblk, vd.size() * 2, hipMemcpyDeviceToHost));
  for (int r = 0; r < n; ++r)
    for (int i = 0; i < HD; ++i) vd[vc_index(pos0 + r, i) - (size_t)b0 * 32 * HD] = V[(size_t)r * HD + i];
  HIPCHK(hipMemcpy(vblk, vd.data(), vd.size() * 2, hipMemcpyHostToDevice));
  return 0;
}

int g4v_model_set_kv(g4v_ctx* c, int l, int pos0, int n, const uint16_t* K, const uint16_t* V) {
  if (!c || (n > 0 && (!K || !V))) return G4V_E_ARG;
  ARGCHK(l >= 0 && l < (int)c->L.size() && pos0 >= 0 && n >= 0 && pos0 + n <= c->ctxcap,
         "model_set_kv: layer or position range outside the cache");
  HIPCHK(hipSetDevice(c->device));
  return kv_upload(c, l, pos0, n, K, V);
}

int g4v_model_fake_ctx(g4v_ctx* c, int n, uint64_t seed) {
  if (!c) return G4V_E_ARG;
  if (!c->model_ready) {
    c->err = "model_fake_ctx: no model";
    return G4V_E_STATE;
  }
  ARGCHK(n >= 0 && n <= c->ctxcap, "model_fake_ctx: n beyond the cache");
  HIPCHK(hipSetDevice(c->device));
  uint32_t rs = (uint32_t)seed;
  auto rnd = [&]() {
    rs = rs * 1664525u + 1013904223u;
    return (float)((int)(rs >> 9) % 2001 - 1000) / 700.0f;
  };
  if (c->gemma) {  // the owner caches of layers 0..14 at their head dims, in the device layouts
    for (int l = 0; l < 15; ++l) {
      const int hd = c->gm[l].hd;
      std::vector<uint16_t> kd((size_t)c->kvcap * hd), vd((size_t)c->kvcap * hd);
      uint16_t* kdev = c->gm_kv.as<uint16_t>() + c->gm_koff[l];
      uint16_t* vdev = c->gm_kv.as<uint16_t>() + c->gm_voff[l];
      HIPCHK(hipMemcpy(kd.data(), kdev, kd.size() * 2, hipMemcpyDeviceToHost));
      HIPCHK(hipMemcpy(vd.data(), vdev, vd.size() * 2, hipMemcpyDeviceToHost));
      for (int p = 0; p < n; ++p)
        for (int e = 0; e < hd; ++e) {  // E:1250: element i = p * hd + e, K then V
          kd[hd == 512 ? kc_index_d<512>(p, e) : kc_index(p, e)] = f2bf(rnd());
          vd[hd == 512 ? vc_index_d<512>(p, e) : vc_index(p, e)] = f2bf(rnd());
        }
      HIPCHK(hipMemcpy(kdev, kd.data(), kd.size() * 2, hipMemcpyHostToDevice));
      HIPCHK(hipMemcpy(vdev, vd.data(), vd.size() * 2, hipMemcpyHostToDevice));
    }
    return 0;
  }
  std::vector<uint16_t> kc((size_t)n * HD), vc((size_t)n * HD);
  for (int l = 0; l < c->NL; ++l) {
    for (size_t i = 0; i < (size_t)n * HD; ++i) {
      kc[i] = f2bf(rnd());
      vc[i] = f2bf(rnd());
    }
    const int r = kv_upload(c, l, 0, n, kc.data(), vc.data());
    if (r) return r;
  }
  return 0;
}

// copies a re-laid int4 matrix back in the reference's [N][K/2] byte layout: row n, chunk c,
// lane j of the device layout holds bytes (j, 8+j) of groups 8c..8c+7
static int read_relaid_w4(g4v_ctx* c, const void* wr, int N, int K, void* dst, size_t cap, size_t* nbytes) {
  const size_t nb = (size_t)N * K / 2;
  if (nbytes) *nbytes = nb;
  if (!dst) return 0;
  ARGCHK(cap >= nb, "model_read: buffer too small");
  std::vector<uint8_t> tmp(nb);
  HIPCHK(hipMemcpy(tmp.data(), wr, nb, hipMemcpyDeviceToHost));
  uint8_t* out = static_cast<uint8_t*>(dst);
  const int GC = K / 256;
  for (size_t n = 0; n < (size_t)N; ++n)
    for (int cc = 0; cc < GC; ++cc)
      for (int jj = 0; jj < 8; ++jj)
        for (int k = 0; k < 8; ++k) {
          const uint8_t* u = tmp.data() + ((n * GC + cc) * 8 + jj) * 16;
          const int g = cc * 8 + k;
          out[n * (K / 2) + g * 16 + jj] = u[2 * k];
          out[n * (K / 2) + g * 16 + 8 + jj] = u[2 * k + 1];
        }
  return 0;
}

int g4v_model_read(g4v_ctx* c, const char* what, void* dst, size_t cap, size_t* nbytes) {
  if (!c || !what) return G4V_E_ARG;
  HIPCHK(hipSetDevice(c->device));
  const void* src = nullptr;
  size_t nb = 0;
  int l = 0, j = 0;
  if (!std::strcmp(what, "E") && c->E.p) {
    src = c->E.p;
    nb = (size_t)c->V * H * 2;
  } else if ((!std::strcmp(what, "KC") || !std::strcmp(what, "VC")) && c->KC.p) {
    // back to the reference's [layer][position][256] rows (positions 0 .. ctxcap - 1)
    const bool key = what[0] == 'K';
    nb = (size_t)c->NL * c->ctxcap * HD * 2;
    if (nbytes) *nbytes = nb;
    if (!dst) return 0;
    ARGCHK(cap >= nb, "model_read: buffer too small");
    std::vector<uint16_t> dev((size_t)c->NL * c->kvcap * HD);
    HIPCHK(hipMemcpy(dev.data(), key ? c->KC.p : c->VC.p, dev.size() * 2, hipMemcpyDeviceToHost));
    uint16_t* o = static_cast<uint16_t*>(dst);
    for (int ll = 0; ll < c->NL; ++ll) {
      const uint16_t* slab = dev.data() + (size_t)ll * c->kvcap * HD;
      for (int p = 0; p < c->ctxcap; ++p)
        for (int e = 0; e < HD; ++e)
          o[((size_t)ll * c->ctxcap + p) * HD + e] = slab[key ? kc_index(p, e) : vc_index(p, e)];
    }
    return 0;
  } else if ((what[0] == 'G' && (what[1] == 'K' || what[1] == 'V')) && c->gemma &&
             std::sscanf(what + 2, "%d", &l) == 1 && l >= 0 && l < 15) {
    // the Gemma layout: owner layer l's cache as the reference's [position][hd] rows
    const bool key = what[1] == 'K';
    const int hd = c->gm[l].hd;
    nb = (size_t)c->ctxcap * hd * 2;
    if (nbytes) *nbytes = nb;
    if (!dst) return 0;
    ARGCHK(cap >= nb, "model_read: buffer too small");
    std::vector<uint16_t> dev((size_t)c->kvcap * hd);
    HIPCHK(hipMemcpy(dev.data(), c->gm_kv.as<uint16_t>() + (key ? c->gm_koff[l] : c->gm_voff[l]), dev.size() * 2,
                     hipMemcpyDeviceToHost));
    uint16_t* o = static_cast<uint16_t*>(dst);
    for (int p = 0; p < c->ctxcap; ++p)
      for (int e = 0; e < hd; ++e)
        o[(size_t)p * hd + e] = dev[hd == 512 ? (key ? kc_index_d<512>(p, e) : vc_index_d<512>(p, e))
                                              : (key ? kc_index(p, e) : vc_index(p, e))];
    return 0;
  } else if (!std::strcmp(what, "fnorm") && c->fnorm.p) {
    src = c->fnorm.p;
    nb = H * 4;
  } else if (!std::strcmp(what, "coef") && c->coef.p) {
    src = c->coef.p;
    nb = (size_t)c->V * 4;
  } else if (!std::strcmp(what, "Sq") && c->scr_s.p) {  // screen scales, [V][48] bf16
    src = c->scr_s.p;
    nb = (size_t)c->V * (H / 32) * 2;
  } else if (!std::strcmp(what, "cb") && c->cb.p) {
    src = c->cb.p;
    nb = 8;
  } else if (!std::strcmp(what, "dec") && c->dec.p) {
    src = c->dec.p;
    nb = (size_t)c->V * H * 2;
  } else if (!std::strcmp(what, "x3sm") && c->x3sm.p) {
    src = c->x3sm.p;
    nb = (size_t)c->V * 24 * 8 * 8;
  } else if (!std::strcmp(what, "x3ix") && c->x3ix.p) {
    src = c->x3ix.p;
    nb = (size_t)c->V * 24 * 8 * 4;
  } else if (!std::strcmp(what, "Wq") && c->scr_wr.p) {  // screen int4, [V][768] bytes
    return read_relaid_w4(c, c->scr_wr.p, c->V, H, dst, cap, nbytes);
  } else if (std::sscanf(what + 1, "%d_%d", &l, &j) == 2 && l >= 0 && l < (int)c->L.size()) {
    const Layer& L = *c->L[l];
    if (what[0] == 'S' && j < 7) {
      src = L.m[j].s.p;
      nb = L.m[j].s.n;
    } else if (what[0] == 'N' && j < 6) {
      src = L.norms.as<float>() + (j < 4 ? j * H : 4 * H + (j - 4) * HD);
      nb = (j < 4 ? H : HD) * 4;
    } else if (what[0] == 'W' && j < 7) {
      const Mat& m = L.m[j];
      return read_relaid_w4(c, m.wr.p, m.N, m.K, dst, cap, nbytes);
    }
  }
  if (!src) {
    c->err = std::string("model_read: unknown array ") + what;
    return G4V_E_ARG;
  }
  if (nbytes) *nbytes = nb;
  if (!dst) return 0;
  ARGCHK(cap >= nb, "model_read: buffer too small");
  HIPCHK(hipMemcpy(dst, src, nb, hipMemcpyDeviceToHost));
  return 0;
}

// ---------------------------------------------------------------------------------------
// verify step
// ---------------------------------------------------------------------------------------
// algorithmic bytes of an int4 G32 matrix read once: N*K/2 weight bytes + N*K/16 scale bytes
static double w4_bytes(const Mat& m) { return (double)m.N * m.K / 2 + (double)m.N * m.K / 16; }

// the attention path of a pass (E:1305 / 1328 / 1337 with SPLITKV, TILED, ATT_PAR = 192):
// 0 split-KV when M <= 4 and pos0 + M > 192, else 1 attn_tile when M >= 4 and pos0 + M > 64 and
// the pass has no sibling row, else 2 run_mh.  One branch row in at most 4 rows is the engine's
// sibling form; larger trees (two branches of several rows, which the engine does not form) take
// the split-KV path for every size
static int pass_path(int M, int pos0, int nb) {
  if (nb > 1 || (nb == 1 && M > 4)) return 0;
  if (M <= 4 && pos0 + M > 192) return 0;
  return (nb == 0 && M >= 4 && pos0 + M > 64) ? 1 : 2;
}

static void enqueue_verify(g4v_ctx* c, int M, int na, int nb, int T, int path) {
  hipStream_t st = c->st;
  const int NL = c->NL, I = c->I;
  // G_I8_ACTIVE in the decode (E:1600) and lin_multi's M >= 2 (E:311): W4A8 products, on the
  // matrices' a8 operand tiles; the same pass otherwise (every other value is exact either way)
  const bool a8 = c->dec_i8 && c->pf_i8 && M >= 2;
  auto a8t = [](const Mat& m) { return W4Tile{m.a8w.as<uint4>(), m.a8s.as<uint4>(), m.N}; };
  const StepDev* sp = c->stepd.as<StepDev>();
  const StepDev& sh = *c->step_host;
  const float sqh = std::sqrt((float)H);
  pmark(c, PT_ROWS, 1, 0);
  launch_embed(c->E.as<uint16_t>(), sp, c->L[0]->ln().in_ln, sqh, c->x.as<float>(), c->xa.as<float>(),
               c->xgs.as<float>(), c->rope.as<float>(), c->ctxcap, c->ropestep.as<float>(), M, st);
  pmark(c, PT_ROWS, 0, (double)M * H * 2);
  for (int l = 0; l < NL; ++l) {
    const Layer& A = *c->L[l];
    const LayerNorms ln = A.ln();
    uint16_t* KCl = c->KC.as<uint16_t>() + (size_t)l * c->kvcap * HD;
    uint16_t* VCl = c->VC.as<uint16_t>() + (size_t)l * c->kvcap * HD;
    // q, k, v in one launch (E:1289)
    GemvTArgs a{};
    for (int j = 0; j < 3; ++j) a.mat[j] = A.m[j].tile();
    a.y[0] = c->q.as<float>();
    a.ldy[0] = NQ * HD;
    a.y[1] = c->k.as<float>();
    a.ldy[1] = HD;
    a.y[2] = c->v.as<float>();
    a.ldy[2] = HD;
    a.K = H;
    a.M = M;
    a.yperm = path == 0 ? 7 : 0;  // the split-KV attention reads q, k, v in the 16-lane head order
    if (l == 0) {  // from the embedding row kernel
      a.xs = c->xa.as<float4>();
      a.gs = c->xgs.as<float>();
    } else {  // the previous layer's MLP residual / norm block (E:1375-1378, E:1390-1404) as prologue
      const LayerNorms pln = c->L[l - 1]->ln();
      a.nrm_mode = 2;
      a.nrm_o = c->o.as<float>();
      a.nrm_xin = c->x2.as<float>();
      a.nrm_xout = c->x.as<float>();
      a.nrm_w1 = pln.post_ff;
      a.nrm_w2 = ln.in_ln;
      a.nrm_scalar = pln.scalar;
    }
    pmark(c, PT_GEMV_QKV, 1, 0);
    if (a8) {
      for (int j = 0; j < 3; ++j) a.mat[j] = a8t(A.m[j]);
      (void)launch_gemv_a8(a, st);
    } else {
      launch_gemv_t(a, st, c->gcfg[0][0], c->gcfg[0][1]);
    }
    pmark(c, PT_GEMV_QKV, 0, w4_bytes(A.m[0]) + w4_bytes(A.m[1]) + w4_bytes(A.m[2]));
    const float* rstep = c->ropestep.as<float>() + (size_t)(A.sliding ? 0 : 1) * MAXM * HD;
    int kmin = sh.pos0 + M - 1;  // E:1325-1326 keys read by the pass: [kmin, pos0 + M - 1]
    for (int r = 0; r < M; ++r) kmin = std::min(kmin, A.sliding ? std::max(0, sh.rope[r] - 511) : 0);
    pmark(c, PT_ATTN, 1, 0);
    if (path == 0) {
      launch_attn(KCl, VCl, c->q.as<float>(), c->k.as<float>(), c->v.as<float>(), ln, rstep, sp, A.sliding, T,
                  c->po.as<float>(), c->pm.as<float>(), c->pl.as<float>(), M, st);
    } else {  // a chain pass below ATT_PAR or of more than 4 rows, or the sibling form below ATT_PAR:
              // the prefill kernels (RoPE position = cache slot = pos0 + m, the sibling's pos0 + 1),
              // output staged for the o projection
      const float* cs = c->rope.as<float>() + (size_t)(2 * (A.sliding ? 0 : 1)) * c->ctxcap * (HD / 2);
      const int sib = nb == 1 ? na + 1 : -1;
      launch_pf_qkv(c->q.as<float>(), c->k.as<float>(), c->v.as<float>(), ln.qn, ln.kn, cs,
                    cs + (size_t)c->ctxcap * (HD / 2), KCl, VCl, sh.pos0, M, st, sib);
      launch_pf_attn(c->q.as<float>(), KCl, VCl, c->vsc.as<float>(), c->vatt.as<float>(),
                     PfGeom{M, sh.pos0, M, sib}, 0, M, A.sliding, st, true);
    }
    pmark(c, PT_ATTN, 0, (double)(sh.pos0 + M - kmin) * HD * 2 * 2);
    pmark(c, PT_GEMV_O, 1, 0);
    GemvTArgs ao{};  // E:1356 on the merged attention (E:1019-1059, formed in the prologue)
    ao.mat[0] = A.m[3].tile();
    ao.y[0] = c->o.as<float>();
    ao.ldy[0] = H;
    if (path == 0 && !a8) {
      ao.mrg_po = c->po.as<float>();
      ao.mrg_pm = c->pm.as<float>();
      ao.mrg_pl = c->pl.as<float>();
      ao.mrg_T = T;
    } else {
      if (path == 0)  // W4A8: the merge on its own (E:1019-1059), staged, then the product
        launch_attn_merge(c->po.as<float>(), c->pm.as<float>(), c->pl.as<float>(), M, T, c->vatt.as<float>(), NQ * HD,
                          c->vags.as<float>(), st, c->q8w.as<uint64_t>(), c->q8s.as<float>());
      ao.xs = c->vatt.as<float4>();  // group sums formed in LDS from the staged copy
    }
    ao.K = NQ * HD;
    ao.M = M;
    if (a8) {
      ao.mat[0] = a8t(A.m[3]);
      if (path == 0) {  // the merge quantised the rows
        ao.xq = c->q8w.as<uint64_t>();
        ao.xqs = c->q8s.as<float>();
      }
      (void)launch_gemv_a8(ao, st);
    } else {
      launch_gemv_t(ao, st, c->gcfg[1][0], c->gcfg[1][1]);
    }
    pmark(c, PT_GEMV_O, 0, w4_bytes(A.m[3]));
    GemvTArgs gu{};  // E:1366 gate/up + gelu, the attention residual / norm block (E:1358-1361) as prologue
    gu.mat[0] = W4Tile{A.m[4].tw.as<uint4>(), A.m[4].ts.as<uint4>(), I};
    gu.gateup = 1;
    gu.y[0] = c->act.as<float>();
    gu.ldy[0] = I;
    gu.nrm_mode = 1;
    gu.nrm_o = c->o.as<float>();
    gu.nrm_xin = c->x.as<float>();
    gu.nrm_xout = c->x2.as<float>();
    gu.nrm_w1 = ln.post_attn;
    gu.nrm_w2 = ln.pre_ff;
    gu.K = H;
    gu.M = M;
    pmark(c, PT_GEMV_GATEUP, 1, 0);
    if (a8) {  // the gate and up matrices' own tiles (the pair-tiled copy is the exact GEMV's)
      gu.mat[0] = a8t(A.m[4]);
      gu.mat[1] = a8t(A.m[5]);
      if (a8_gateup_quantises(I)) {  // the activation quantised for down by the same blocks
        gu.yq = c->q8w.as<uint64_t>();
        gu.yqs = c->q8s.as<float>();
      }
      (void)launch_gemv_a8(gu, st);
    } else {
      launch_gemv_t(gu, st, c->gcfg[2][0], c->gcfg[2][1]);
    }
    pmark(c, PT_GEMV_GATEUP, 0, w4_bytes(A.m[4]) + w4_bytes(A.m[5]));
    pmark(c, PT_GEMV_DOWN, 1, 0);
    GemvTArgs ad{};  // E:1373
    ad.mat[0] = A.m[6].tile();
    ad.y[0] = c->o.as<float>();
    ad.ldy[0] = H;
    ad.xs = c->act.as<float4>();  // group sums formed in LDS from the staged copy
    ad.K = I;
    ad.M = M;
    if (a8) {
      ad.mat[0] = a8t(A.m[6]);
      if (a8_gateup_quantises(I)) {
        ad.xq = c->q8w.as<uint64_t>();
        ad.xqs = c->q8s.as<float>();
      }
      (void)launch_gemv_a8(ad, st);
    } else {
      launch_gemv_t(ad, st, I > 6144 ? 1 : c->gcfg[3][0], c->gcfg[3][1]);  // (K 12288: one row per block)
    }
    pmark(c, PT_GEMV_DOWN, 0, w4_bytes(A.m[6]));
    if (l + 1 == NL) {  // the last MLP residual block and the final norm (E:1414-1417) for the head
      pmark(c, PT_ROWS, 1, 0);
      launch_post_ff(c->o.as<float>(), c->x2.as<float>(), c->xa.as<float>(), c->xgs.as<float>(), ln, nullptr,
                     c->fnorm.as<float>(), c->h.as<float>(), c->hn.as<float>(), M, st);
      pmark(c, PT_ROWS, 0, (double)M * H * 4 * 4);
    }
  }
  // head of row 0, then of the branch its token selects (E:1475-1488)
  HeadRun h1 = head_args(c, c->hb1, c->h.as<float>(), c->hn.as<float>(), 1, nullptr);
  head_run(h1, st);
  VerifyResultDev* res = c->resd.as<VerifyResultDev>();
  pmark(c, PT_ACCEPT, 1, 0);
  launch_branch(sp, c->hb1.hs.best, c->h.as<float>(), c->hn.as<float>(), c->h2.as<float>(), c->hn2.as<float>(), res,
                st);
  pmark(c, PT_ACCEPT, 0, 0);
  const int M2 = std::max(1, std::max(na, nb));
  HeadRun h2 = head_args(c, c->hb2, c->h2.as<float>(), c->hn2.as<float>(), M2, &res->hcount);
  h2.pass2 = 1;
  head_run(h2, st);
  pmark(c, PT_ACCEPT, 1, 0);
  launch_accept(sp, c->hb1.hs.best, c->hb2.hs.best, c->hb1.hs.cnt, c->hb2.hs.cnt, res, c->KC.as<uint16_t>(),
                c->VC.as<uint16_t>(), NL, c->kvcap, st);
  pmark(c, PT_ACCEPT, 0, 0);
}

static int verify_pass(g4v_ctx* c, const int* toks, int na, int nb, int pos0, int nsplit, int b_ok,
                       g4v_verify_result* out, float* hidden);
static int gm_verify(g4v_ctx* c, const int* toks, int na, int nb, int pos0, int nsplit, int b_ok,
                     g4v_verify_result* out, float* hidden);

int g4v_verify_step(g4v_ctx* c, const int* toks, int na, int nb, int pos0, int nsplit, g4v_verify_result* out,
                    float* hidden) {
  return verify_pass(c, toks, na, nb, pos0, nsplit, 1, out, hidden);
}

int g4v_verify_sibling(g4v_ctx* c, const int* toks, int nd, int pos0, int nsplit, int allow_hit,
                       g4v_verify_result* out, float* hidden) {
  if (!c) return G4V_E_ARG;
  ARGCHK(nd >= 1 && nd <= 2, "verify_sibling: 1 <= nd <= 2 (the sibling form has at most 4 rows)");
  return verify_pass(c, toks, nd, 1, pos0, nsplit, allow_hit ? 1 : 0, out, hidden);
}

static int verify_pass(g4v_ctx* c, const int* toks, int na, int nb, int pos0, int nsplit, int b_ok,
                       g4v_verify_result* out, float* hidden) {
  if (c && c->gemma) return gm_verify(c, toks, na, nb, pos0, nsplit, b_ok, out, hidden);
  if (!c) return G4V_E_ARG;
  std::string missing;
  if (!c->model_ready || !model_complete(c, &missing)) {
    c->err = "verify_step: model incomplete: " + (c->model_ready ? missing : std::string("no model"));
    return G4V_E_STATE;
  }
  const int M = 1 + na + nb;
  // a chain of up to 7 drafts (E:1514 ENGINE_NGLEN <= 7, M <= 8 rows through attn_tile or run_mh,
  // E:1328-1349), or a tree of two branches of up to 4 drafts each
  ARGCHK(toks && out && na >= 0 && nb >= 0 && M <= MAXM && ((nb == 0 && na <= 7) || (na <= 4 && nb <= 4)),
         "verify_step: a chain of 0 <= na <= 7 drafts, or 0 <= na, nb <= 4");
  ARGCHK(nb == 0 || na >= 1, "verify_step: branch b needs a chain a");
  ARGCHK(pos0 >= 1 && pos0 + M <= c->ctxcap, "verify_step: positions beyond the cache");
  ARGCHK(nsplit >= 1 && nsplit <= MAXT, "verify_step: 1 <= nsplit <= 16");
  ARGCHK((pos0 + M + nsplit - 1) / nsplit + 1 <= attn_pmax(), "verify_step: context too long for nsplit");
  for (int i = 0; i < M; ++i) ARGCHK(toks[i] >= 0 && toks[i] < c->V, "verify_step: token id out of range");
  HIPCHK(hipSetDevice(c->device));
  StepDev& s = *c->step_host;
  std::memset(&s, 0, sizeof s);
  s.M = M;
  s.na = na;
  s.nb = nb;
  s.pos0 = pos0;
  s.b_ok = b_ok;
  for (int r = 0; r < M; ++r) {
    s.toks[r] = toks[r];
    if (r <= na) {
      s.rope[r] = pos0 + r;
      s.skip_lo[r] = 1;
      s.skip_hi[r] = 0;
    } else {  // branch b: RoPE position by depth, skip chain a's slots (E:1292, 1326)
      s.rope[r] = pos0 + (r - na);
      s.skip_lo[r] = pos0 + 1;
      s.skip_hi[r] = pos0 + na;
    }
  }
  const int path = pass_path(M, pos0, nb);
  const bool a8 = c->dec_i8 && c->pf_i8 && M >= 2;  // the pass's products (enqueue_verify)
  const long long key = (((((long long)M * 8 + na) * 8 + nb) * 32 + nsplit) * 2 + (a8 ? 1 : 0)) * 65536 + c->prof_mask;
  g4v_ctx::Graph* gr = nullptr;
  for (auto& g : c->graphs)
    if (g.key == key && path == 0) gr = &g;  // only split-KV passes are captured
  const bool warm = std::find(c->warmed.begin(), c->warmed.end(), key) != c->warmed.end();
  if (gr) {  // replay: the pinned step block is copied in by the graph's first node
    HIPCHK(hipGraphLaunch(gr->exec, c->st));
  } else if (!c->use_graph || !warm || path != 0) {  // eager (first call of a shape, graphs disabled, or
                                                     // a pass whose attention kernels take pos0 as an argument)
    HIPCHK(hipMemcpyAsync(c->stepd.p, &s, sizeof s, hipMemcpyHostToDevice, c->st));
    enqueue_verify(c, M, na, nb, nsplit, path);
    HIPCHK(hipGetLastError());
    HIPCHK(hipMemcpyAsync(c->res_host, c->resd.p, sizeof(VerifyResultDev), hipMemcpyDeviceToHost, c->st));
    c->step_events = c->evused;  // profiling events one pass of this shape needs
    if (!warm) c->warmed.push_back(key);
  } else {  // capture the whole pass once, then launch it
    g4v_ctx::Graph g;
    g.key = key;
    const size_t ev0 = c->evpool.size();
    for (size_t k = 0; k < c->step_events; ++k) {  // no event may be created while capturing
      hipEvent_t e;
      HIPCHK(hipEventCreate(&e));
      c->evpool.push_back(e);
    }
    c->evused = ev0;  // the graph's profiling nodes use the fresh events
    c->recs.clear();
    hipGraph_t graph;
    HIPCHK(hipStreamBeginCapture(c->st, hipStreamCaptureModeThreadLocal));
    (void)hipMemcpyAsync(c->stepd.p, &s, sizeof s, hipMemcpyHostToDevice, c->st);
    enqueue_verify(c, M, na, nb, nsplit, 0);
    (void)hipMemcpyAsync(c->res_host, c->resd.p, sizeof(VerifyResultDev), hipMemcpyDeviceToHost, c->st);
    HIPCHK(hipStreamEndCapture(c->st, &graph));
    const hipError_t ei = hipGraphInstantiate(&g.exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (ei != hipSuccess) {
      c->err = std::string("hipGraphInstantiate: ") + hipGetErrorString(ei);
      return G4V_E_HIP;
    }
    g.events.assign(c->evpool.begin() + ev0, c->evpool.end());
    c->evpool.resize(ev0);
    c->evused = 0;
    g.recs = c->recs;
    c->recs.clear();
    c->graphs.push_back(std::move(g));
    gr = &c->graphs.back();
    HIPCHK(hipGraphLaunch(gr->exec, c->st));
  }
  HIPCHK(hipStreamSynchronize(c->st));
  const VerifyResultDev& r = *c->res_host;
  if (c->prof_mask) {
    if (gr) c->recs = gr->recs;  // the graph re-records the same events on every launch
    prof_collect(c, r.fallback[0] != 0);
  }
  out->nacc = r.nacc;
  out->branch = r.branch;
  out->ncommit = r.ncommit;
  for (int i = 0; i < 8; ++i) {
    out->commit[i] = r.commit[i];
    out->G[i] = r.G[i];
    out->fallback[i] = r.fallback[i];
    out->nsurv[i] = r.nsurv[i];
  }
  c->last_hrow = r.hrows[r.ncommit - 1];
  if (hidden)
    HIPCHK(hipMemcpy(hidden, c->h.as<float>() + (size_t)c->last_hrow * H, H * 4, hipMemcpyDeviceToHost));
  return 0;
}


// ---------------------------------------------------------------------------------------
// prefill
// ---------------------------------------------------------------------------------------
// a linear layer of a prefill segment: lin_multi / lin1 (E:310-317) take W4A8 when the block has
// M >= 2 rows (G_I8_ACTIVE during prefill), else the exact-float GEMV.  quant = false reuses the
// quantised rows of the previous call (same x).
static void pf_lin(g4v_ctx* c, const Mat& m, const float* x, int M, float* y, bool i8, bool quant) {
  if (i8) {
    if (quant)
      launch_w4a8_quant(x, M, w4a8_mpad(M), m.K, c->pfxq.as<uint16_t>(), c->pfsx.as<float>(), c->pfcorr.as<float>(),
                        nullptr, nullptr, nullptr, c->st);
    launch_w4a8_gemm(m.a8w.as<uint4>(), m.a8s.as<uint4>(), c->pfxq.as<uint16_t>(), c->pfsx.as<float>(),
                     c->pfcorr.as<float>(), y, M, m.N, m.K, m.N, c->st);
  } else {  // the exact-float GEMV, MAXM rows a launch (each row's result is independent of the others)
    for (int r = 0; r < M; r += MAXM)
      launch_gemv(plain_args(m, x + (size_t)r * m.K, y + (size_t)r * m.N, std::min(MAXM, M - r)), EPI_STORE, c->st);
  }
}

// up to three products of the same input (same K) in one launch per MAXM rows: q / k / v, gate / up
static void pf_lin_multi(g4v_ctx* c, int n, const Mat* const* m, const float* x, int M, float* const* y, bool i8) {
  if (i8) {
    bool n16 = true;
    for (int j = 0; j < n; ++j) n16 = n16 && m[j]->N % 16 == 0;
    if (M <= 8 && n16) {  // decode rows: the n products in one launch (i8_task over nj matrices, E:303-309)
      launch_w4a8_quant(x, M, w4a8_mpad(M), m[0]->K, c->pfxq.as<uint16_t>(), c->pfsx.as<float>(),
                        c->pfcorr.as<float>(), nullptr, nullptr, nullptr, c->st);
      A8Dec d{};
      for (int j = 0; j < n; ++j) {
        d.tw[j] = m[j]->a8w.as<uint4>();
        d.ts[j] = m[j]->a8s.as<uint4>();
        d.y[j] = y[j];
        d.ldy[j] = m[j]->N;
        d.t0[j + 1] = d.t0[j] + m[j]->N / 16;
      }
      for (int j = n + 1; j < 4; ++j) d.t0[j] = d.t0[n];
      if (launch_w4a8_dec(d, n, c->pfxq.as<uint16_t>(), c->pfsx.as<float>(), c->pfcorr.as<float>(), M, m[0]->K,
                          c->st))
        return;
    }
    for (int j = 0; j < n; ++j) pf_lin(c, *m[j], x, M, y[j], true, j == 0);
    return;
  }
  const int K = m[0]->K;
  for (int r = 0; r < M; r += MAXM) {
    GemvArgs a{};
    for (int j = 0; j < n; ++j) {
      a.mat[j] = m[j]->dev();
      a.y[j] = y[j] + (size_t)r * m[j]->N;
      a.ldy[j] = m[j]->N;
    }
    a.x = x + (size_t)r * K;
    a.ldx = K;
    a.K = K;
    a.M = std::min(MAXM, M - r);
    launch_gemv(a, EPI_STORE, c->st);
  }
}

static int pf_alloc(g4v_ctx* c, int rows, size_t sfl) {
  if (rows > c->pf_rows || c->I != c->pf_I) {
    const size_t R = (size_t)rows, Rp = (size_t)w4a8_mpad(rows), Kmax = std::max(NQ * HD, std::max(H, c->I));
    ALLOC(c->pfx, R * H * 4);
    ALLOC(c->pfa, R * H * 4);
    ALLOC(c->pfq, R * NQ * HD * 4);
    ALLOC(c->pfk, R * HD * 4);
    ALLOC(c->pfv, R * HD * 4);
    ALLOC(c->pfatt, R * NQ * HD * 4);
    ALLOC(c->pfo, R * H * 4);
    ALLOC(c->pfg, R * c->I * 4);
    ALLOC(c->pfu, R * c->I * 4);
    ALLOC(c->pfact, R * c->I * 4);
    ALLOC(c->pfxq, Rp * Kmax * 2);
    ALLOC(c->pfsx, (Kmax / 32) * Rp * 4);
    ALLOC(c->pfcorr, (Kmax / 32) * Rp * 4);
    ALLOC(c->pftok, R * 4);
    if (!c->pfh.p) ALLOC(c->pfh, H * 4);
    c->pf_rows = rows;
    c->pf_I = c->I;
  }
  if (sfl > c->pf_sfl) {
    ALLOC(c->pfs, sfl * 4);
    c->pf_sfl = sfl;
  }
  return 0;
}

// rows [r0, r0 + M) of the prompt through every layer.  split: the rows form one short block that
// takes the split-KV path (E:1305) with nsplit splits; else each row takes attn_tile or run_mh
// by its block.  After the last layer, h = the final-normed state of segment row hrow (or none).
static void pf_segment(g4v_ctx* c, const PfGeom& g, int r0, int M, bool i8, bool split, int nsplit, int hrow) {
  hipStream_t st = c->st;
  const float sqh = std::sqrt((float)H);
  const size_t off = (size_t)r0;
  float *x = c->pfx.as<float>() + off * H, *a = c->pfa.as<float>() + off * H, *o = c->pfo.as<float>() + off * H;
  float *q = c->pfq.as<float>() + off * NQ * HD, *k = c->pfk.as<float>() + off * HD, *v = c->pfv.as<float>() + off * HD;
  float* att = c->pfatt.as<float>() + off * NQ * HD;
  float *gb = c->pfg.as<float>() + off * c->I, *ub = c->pfu.as<float>() + off * c->I,
        *act = c->pfact.as<float>() + off * c->I;
  const int P0 = g.pos0 + r0;
  launch_pf_embed(c->E.as<uint16_t>(), c->pftok.as<int>() + r0, c->L[0]->ln().in_ln, sqh, x, a, M, st);
  for (int l = 0; l < c->NL; ++l) {
    const Layer& lay = *c->L[l];
    const LayerNorms ln = lay.ln();
    const int ty = lay.sliding ? 0 : 1;
    uint16_t* KCl = c->KC.as<uint16_t>() + (size_t)l * c->kvcap * HD;
    uint16_t* VCl = c->VC.as<uint16_t>() + (size_t)l * c->kvcap * HD;
    pf_lin(c, lay.m[0], a, M, q, i8, true);  // E:1289
    pf_lin(c, lay.m[1], a, M, k, i8, false);
    pf_lin(c, lay.m[2], a, M, v, i8, false);
    const float* cs = c->rope.as<float>() + (size_t)(2 * ty) * c->ctxcap * (HD / 2);
    const float* sn = cs + (size_t)c->ctxcap * (HD / 2);
    launch_pf_qkv(q, k, v, ln.qn, ln.kn, cs, sn, KCl, VCl, P0, M, st);
    if (split) {  // E:1305-1327: one block of M <= 4 rows over [kmin, kmax]
      AttnGeom ag{};
      ag.M = M;
      ag.kmax = P0 + M - 1;
      ag.kmin = ag.kmax;
      ag.T = nsplit;
      for (int m = 0; m < M; ++m) {
        ag.pos[m] = P0 + m;
        ag.lo[m] = lay.sliding ? std::max(0, P0 + m - 511) : 0;
        ag.skip_lo[m] = 1;
        ag.skip_hi[m] = 0;
        ag.kmin = std::min(ag.kmin, ag.lo[m]);
      }
      launch_attn_geom(KCl, VCl, q, NQ * HD, ag, c->po.as<float>(), c->pm.as<float>(), c->pl.as<float>(), att,
                       NQ * HD, st);
    } else {
      launch_pf_attn(c->pfq.as<float>(), KCl, VCl, c->pfs.as<float>(), c->pfatt.as<float>(), g, r0, M, lay.sliding,
                     st);
    }
    pf_lin(c, lay.m[3], att, M, o, i8, true);  // E:1356
    launch_pf_post_attn(o, x, a, ln.post_attn, ln.pre_ff, M, st);
    pf_lin(c, lay.m[4], a, M, gb, i8, true);  // E:1366-1371
    pf_lin(c, lay.m[5], a, M, ub, i8, false);
    launch_pf_act(gb, ub, act, (size_t)M * c->I, st);
    pf_lin(c, lay.m[6], act, M, o, i8, true);  // E:1373
    const bool lastl = l + 1 == c->NL;
    launch_pf_post_ff(o, x, a, ln.post_ff, lastl ? nullptr : c->L[l + 1]->ln().in_ln, c->fnorm.as<float>(),
                      lay.scalar, c->pfh.as<float>(), lastl ? hrow : -1, M, st);
  }
}

// ---------------------------------------------------------------------------------------
// The Gemma-4-E2B layer layout (E:1222-1232, fwd E:1256-1405): 35 layers of head dim 256
// (l % 5 != 4, window 512) or 512 (global: RoPE theta 1e6 on the first quarter of the
// frequencies, E:1246-1247), k / v projections and caches in layers 0..14 only (layer l >= 15
// reads the cache of layer 13 or 14, E:1251), each layer's MLP width, and the per-layer-input
// branch (ple_fused_task E:615-660 once per pass, pg_fused_task E:405-443 + per_layer_projection
// + post_per_layer_input_norm per layer, E:1379-1404).  A pass of M <= 32 rows runs as the
// prefill path runs a block (plain row layouts, the exact-float GEMV or, for prompt blocks with
// g4v_set_prefill_int8, W4A8), eagerly; the head and acceptance are the verify pass's own.
// ---------------------------------------------------------------------------------------
}  // extern "C"

namespace {
constexpr int GM_NL = 35, GM_PD = 256, GM_ROWS = 32, GM_PLN = GM_NL * GM_PD;
int gm_hd(int l) { return l % 5 != 4 ? 256 : 512; }
int gm_owner(int l) { return l < 15 ? l : (l % 5 != 4 ? 13 : 14); }  // E:1251

struct GmRows {
  float *x, *a, *o, *q, *k, *v, *att, *g, *u, *act, *pr, *pli, *pgv, *g2;
};
GmRows gm_rows(g4v_ctx* c) {
  float* f = c->gm_rows.as<float>();
  const size_t R = c->gm_cap, I = c->gm_Imax;
  GmRows r;
  r.x = f;
  r.a = r.x + R * H;
  r.o = r.a + R * H;
  r.q = r.o + R * H;
  r.k = r.q + R * NQ * 512;
  r.v = r.k + R * 512;
  r.att = r.v + R * 512;
  r.g = r.att + R * NQ * 512;
  r.u = r.g + R * I;
  r.act = r.u + R * I;
  r.pr = r.act + R * I;
  r.pli = r.pr + R * GM_PLN;
  r.pgv = r.pli + R * GM_PLN;
  r.g2 = r.pgv + R * GM_PD;
  return r;
}
size_t gm_rows_floats(int Imax, int rows) {
  const size_t R = rows;
  return R * (3 * H + 2 * NQ * 512 + 2 * 512 + 3 * (size_t)Imax + 2 * GM_PLN + 2 * GM_PD);
}

// row buffers, token slots and W4A8 operands for passes of up to `rows` rows, score scratch of
// `sfl` floats (grown, never shrunk)
int gm_reserve(g4v_ctx* c, int rows, size_t sfl) {
  if (rows > c->gm_cap || sfl > c->gm_sfl) drop_graphs(c);  // captured passes hold these buffers
  if (rows > c->gm_cap) {
    ALLOC(c->gm_rows, gm_rows_floats(c->gm_Imax, rows) * 4);
    ALLOC(c->gm_tok, (size_t)rows * 4);
    const size_t Kmax = std::max<size_t>(NQ * 512, std::max<size_t>(H, c->gm_Imax)), Rp = (size_t)w4a8_mpad(rows);
    ALLOC(c->pfxq, Rp * Kmax * 2);
    ALLOC(c->pfsx, (Kmax / 32) * Rp * 4);
    ALLOC(c->pfcorr, (Kmax / 32) * Rp * 4);
    c->gm_cap = rows;
  }
  if (sfl > c->gm_sfl) {
    ALLOC(c->gm_s, sfl * 4);
    c->gm_sfl = sfl;
  }
  return 0;
}

// matrix j of layer l: 0 q, 1 k, 2 v, 3 o, 4 gate, 5 up, 6 down, 7 per_layer_input_gate, 8 per_layer_projection
void gm_shape(const g4v_ctx* c, int l, int j, int* N, int* K) {
  const int hd = gm_hd(l), I = c->gm[l].I;
  const int n[9] = {NQ * hd, hd, hd, H, I, I, H, GM_PD, H}, k[9] = {H, H, H, NQ * hd, H, H, I, H, GM_PD};
  *N = n[j];
  *K = k[j];
}
Mat& gm_mat(g4v_ctx* c, int l, int j) { return j < 7 ? c->L[l]->m[j] : (j == 7 ? c->gm[l].pg : c->gm[l].pp); }
// the matrices the verify pass multiplies with the row-tile GEMV (row-tiled copies): all but gate
// and up (paired by tile_gateup)
bool gm_tiled(int j, int K) { return j != 4 && j != 5 && K <= 12288; }

bool gm_complete(const g4v_ctx* c, std::string* what) {
  if (!c->head_ready) {
    *what = "embedding / head not set";
    return false;
  }
  if (!c->gm_plready) {
    *what = "per_layer_model_projection not set";
    return false;
  }
  for (int l = 0; l < GM_NL; ++l) {
    for (int j = 0; j < 9; ++j)
      if ((j != 1 && j != 2) || c->gm[l].own)
        if (!gm_mat(const_cast<g4v_ctx*>(c), l, j).wr.p) {
          *what = "matrix " + std::to_string(j) + " of layer " + std::to_string(l) + " not set";
          return false;
        }
    if (!c->gm[l].normed) {
      *what = "norms of layer " + std::to_string(l) + " not set";
      return false;
    }
  }
  return true;
}

// fwd (E:1256-1405) of the M rows whose tokens are in gm_tok, at positions pos0 .. pos0 + M - 1,
// row sib (>= 0) the sibling row (E:1292, 1340-1345); i8: W4A8 linear layers (M >= 2).  Rows
// m >= hrow (hrow >= 0) leave their final-normed state in h [M - hrow][1536] and |h| in hn.
// pg: the rows are a run of whole prompt blocks (pg->pfb rows each, at least 5): each block's
// rows take that block's attention path (attn_tile or run_mh, E:1328-1337), in one pass.
// spd not null (a verify pass): the rows' tokens and positions are read from the step parameters
// on the device (pos0 here only picks the attention path), so that the pass can be captured once
// and replayed at any position
void gm_forward(g4v_ctx* c, int M, int pos0, int nsplit, int sib, int hrow, bool i8, float* h, float* hn,
                const PfGeom* pg = nullptr, const StepDev* spd = nullptr) {
  hipStream_t st = c->st;
  const GmRows R = gm_rows(c);
  const float sqh = std::sqrt((float)H);
  const int* tok = spd ? spd->toks : c->gm_tok.as<int>();
  const int* dpos = spd ? &spd->pos0 : nullptr;
  const bool split = !pg && M <= 4 && pos0 + M > 192;  // E:1305-1327
  AttnGeom* geo = c->gm_geo.as<AttnGeom>();
  if (spd && split) launch_step_geom(spd, nsplit, geo, st);
  i8 = i8 && M >= 2;  // lin_multi's rule (E:311)
  launch_pf_embed(c->E.as<uint16_t>(), tok, c->gm[0].nv.as<float>(), sqh, R.x, R.a, M, st);  // E:1262-1267
  pf_lin(c, c->gm_plproj, R.x, M, R.pr, i8, true);                                            // E:615-660
  launch_gm_ple(R.pr, tok, c->gm_ple.as<uint16_t>(), c->gm_plnorm.as<float>(), R.pli, M, st);
  for (int l = 0; l < GM_NL; ++l) {
    const auto& G = c->gm[l];
    const Layer& lay = *c->L[l];
    const int hd = G.hd, ty = hd == 512, own = G.own, ol = gm_owner(l);
    const bool sliding = !ty;
    const float* nv = G.nv.as<float>();
    const float *in_ln = nv, *post_attn = nv + H, *pre_ff = nv + 2 * H, *post_ff = nv + 3 * H, *post_ple = nv + 4 * H,
                *qn = nv + 5 * H, *kn = nv + 5 * H + hd;
    (void)in_ln;
    uint16_t* KCo = c->gm_kv.as<uint16_t>() + c->gm_koff[ol];
    uint16_t* VCo = c->gm_kv.as<uint16_t>() + c->gm_voff[ol];
    {  // E:1287-1288: q (and k, v on the owner layers) in one launch
      const Mat* mq[3] = {&lay.m[0], &lay.m[1], &lay.m[2]};
      float* yq[3] = {R.q, R.k, R.v};
      pf_lin_multi(c, own ? 3 : 1, mq, R.a, M, yq, i8);
    }
    const float* cs = ty ? c->gm_rope.as<float>() : c->rope.as<float>();
    const float* sn = cs + (size_t)c->ctxcap * (hd / 2);
    launch_pf_qkv(R.q, R.k, R.v, qn, kn, cs, sn, KCo, VCo, pos0, M, st, sib, hd, own, dpos);
    if (split) pmark(c, PT_ATTN, 1, 0);  // the split-KV attention (E:1327 T_ATT)
    if (split && spd) {
      if (hd == 512)
        launch_attn_geom_dev_hd(KCo, VCo, R.q, NQ * 512, geo + ty, M, nsplit, NQ, c->po5.as<float>(),
                                c->pm5.as<float>(), c->pl5.as<float>(), R.att, NQ * 512, st);
      else
        launch_attn_geom_dev(KCo, VCo, R.q, NQ * HD, geo + ty, M, nsplit, c->po.as<float>(), c->pm.as<float>(),
                             c->pl.as<float>(), R.att, NQ * HD, st);
    } else if (split) {
      AttnGeom ag{};
      ag.M = M;
      ag.kmax = pos0 + M - 1;
      ag.kmin = ag.kmax;
      ag.T = nsplit;
      for (int m = 0; m < M; ++m) {
        const int rp = m == sib ? pos0 + 1 : pos0 + m;
        ag.pos[m] = pos0 + m;
        ag.lo[m] = sliding ? std::max(0, rp - 511) : 0;
        ag.skip_lo[m] = m == sib ? pos0 + 1 : 1;
        ag.skip_hi[m] = m == sib ? pos0 + m - 1 : 0;
        ag.kmin = std::min(ag.kmin, ag.lo[m]);
      }
      if (hd == 512)
        (void)launch_attn_geom_hd(KCo, VCo, R.q, NQ * 512, ag, 512, c->po5.as<float>(), c->pm5.as<float>(),
                                  c->pl5.as<float>(), R.att, NQ * 512, nullptr, st);
      else
        launch_attn_geom(KCo, VCo, R.q, NQ * HD, ag, c->po.as<float>(), c->pm.as<float>(), c->pl.as<float>(), R.att,
                         NQ * HD, st);
    } else {  // attn_tile (M >= 4 past 64 keys, no sibling) or run_mh: one block of M rows
      launch_pf_attn(R.q, KCo, VCo, c->gm_s.as<float>(), R.att, pg ? *pg : PfGeom{M, pos0, M, sib}, 0, M, sliding,
                     st, false, hd, dpos, c->ctxcap);
    }
    if (split) pmark(c, PT_ATTN, 0, 0);
    pf_lin(c, lay.m[3], R.att, M, R.o, i8, true);                       // E:1356
    launch_pf_post_attn(R.o, R.x, R.a, post_attn, pre_ff, M, st);       // E:1358-1361
    {  // E:1363-1371: gate and up in one launch
      const Mat* mg[2] = {&lay.m[4], &lay.m[5]};
      float* yg[2] = {R.g, R.u};
      pf_lin_multi(c, 2, mg, R.a, M, yg, i8);
    }
    launch_pf_act(R.g, R.u, R.act, (size_t)M * G.I, st);
    pf_lin(c, lay.m[6], R.act, M, R.o, i8, true);                                               // E:1373
    launch_pf_post_ff(R.o, R.x, R.a, post_ff, nullptr, nullptr, 1.0f, nullptr, -1, M, st);      // E:1375-1377
    pf_lin(c, G.pg, R.x, M, R.pgv, i8, true);                                                   // E:1379-1384
    launch_gm_pg_act(R.pgv, R.pli, l, M, R.g2, st);
    pf_lin(c, G.pp, R.g2, M, R.o, i8, true);                                                    // E:1386
    const bool last = l + 1 == GM_NL;                                                           // E:1387-1404
    launch_pf_post_ff(R.o, R.x, R.a, post_ple, last ? nullptr : c->gm[l + 1].nv.as<float>(), c->fnorm.as<float>(),
                      G.scalar, h, last ? hrow : -1, M, st, hn);
  }
}

// fwd of a verify pass (M <= MAXM rows, exact float) with the row-tile GEMV: every residual / norm
// block folded into the prologue of the product that consumes it, as the synthetic stack's
// verify pass does.  Per layer: q/k/v (prologue: the previous layer's per-layer-input residual,
// scalar and input norm, E:1390-1404), q/k norm + RoPE + cache rows, attention (split-KV past
// ATT_PAR for up to 4 rows, else attn_tile / run_mh, output staged), o, gate/up + gelu
// (prologue: attention residual and pre-FF norm, E:1358-1361), down, the per-layer-input gate
// (prologue: the MLP residual, E:1375-1377; epilogue: gelu x per-layer input, E:1379-1385) and
// its projection (E:1386).  Residual rows: xa at a layer's start, xb after attention, xc after
// the MLP (R.x, R.a, R.g); the products' outputs meet their consumers in R.o.  The last row
// block's final-normed state goes to h / hn (row 0 on).
// a8 (G_I8_ACTIVE in the decode, 2 <= M <= 8): every product multiplies W4A8 (lin_multi, E:310-317)
// through the same structure -- the W4A8 kernel takes the same prologues and epilogues and
// quantises its activation rows itself -- so the values that reach the products are the ones the
// exact pass forms, as in the reference, where only lin_multi's branch differs (E:1268-1289,
// 1363-1388 compute the same rows in either mode).
void gm_verify_forward(g4v_ctx* c, int M, int pos0, int nsplit, int sib, float* h, float* hn, const StepDev* spd,
                       bool a8 = false) {
  hipStream_t st = c->st;
  const GmRows R = gm_rows(c);
  const int* dpos = spd ? &spd->pos0 : nullptr;
  const bool split = M <= 4 && pos0 + M > 192;  // E:1305-1327
  AttnGeom* geo = c->gm_geo.as<AttnGeom>();
  if (spd && split) launch_step_geom(spd, nsplit, geo, st);
  float *xa = R.x, *xb = R.a, *xc = R.g, *attgs = R.u;
  // a one-row pass runs 32-row tiles (twice the blocks of a 64-row tile: one subset only)
  auto rows_of = [&](int cls) { return M == 1 ? 1 : c->gcfg[cls][0]; };
  auto tile_of = [&](int cls) { return M == 1 ? 32 : c->gcfg[cls][1]; };
  a8 = a8 && M >= 2;  // lin_multi's rule (E:311)
  // a product: the W4A8 kernel on the a8 tiles of the same matrices, or the row-tile GEMV
  auto a8t = [](const Mat& m) { return W4Tile{m.a8w.as<uint4>(), m.a8s.as<uint4>(), m.N}; };
  auto product = [&](GemvTArgs& a, const Mat* const* ms, int nm, int mpl, int tr) {
    if (a8) {
      for (int j = 0; j < nm; ++j) a.mat[j] = a8t(*ms[j]);
      (void)launch_gemv_a8(a, st);
    } else {
      (void)launch_gemv_t(a, st, mpl, tr);
    }
  };
  const float sqh = std::sqrt((float)H);
  const int* tok = spd ? spd->toks : c->gm_tok.as<int>();
  launch_pf_embed(c->E.as<uint16_t>(), tok, c->gm[0].nv.as<float>(), sqh, xa, xb, M, st);  // E:1262-1267
  pf_lin(c, c->gm_plproj, xa, M, R.pr, a8, true);                                          // E:615-660
  launch_gm_ple(R.pr, tok, c->gm_ple.as<uint16_t>(), c->gm_plnorm.as<float>(), R.pli, M, st);
  for (int l = 0; l < GM_NL; ++l) {
    const auto& G = c->gm[l];
    const Layer& lay = *c->L[l];
    const int hd = G.hd, own = G.own, ol = gm_owner(l);
    const bool sliding = hd != 512;
    const float* nv = G.nv.as<float>();
    const float *post_attn = nv + H, *pre_ff = nv + 2 * H, *post_ff = nv + 3 * H, *qn = nv + 5 * H, *kn = nv + 5 * H + hd;
    uint16_t* KCo = c->gm_kv.as<uint16_t>() + c->gm_koff[ol];
    uint16_t* VCo = c->gm_kv.as<uint16_t>() + c->gm_voff[ol];
    if (l == 0) {  // E:1287-1288 from the embedding row's norm
      const Mat* mq[3] = {&lay.m[0], &lay.m[1], &lay.m[2]};
      float* yq[3] = {R.q, R.k, R.v};
      pf_lin_multi(c, own ? 3 : 1, mq, xb, M, yq, a8);
    } else {
      const auto& P = c->gm[l - 1];
      const float* pnv = P.nv.as<float>();
      GemvTArgs a{};
      const int nm = own ? 3 : 1;
      float* ys[3] = {R.q, R.k, R.v};
      const int ld[3] = {NQ * hd, hd, hd};
      for (int j = 0; j < nm; ++j) {
        a.mat[j] = lay.m[j].tile();
        a.y[j] = ys[j];
        a.ldy[j] = ld[j];
      }
      a.K = H;
      a.M = M;
      a.nrm_mode = 2;
      a.nrm_o = R.o;
      a.nrm_xin = xc;
      a.nrm_xout = xa;
      a.nrm_w1 = pnv + 4 * H;  // post_per_layer_input_norm of layer l - 1
      a.nrm_w2 = nv;           // input_layernorm of layer l
      a.nrm_scalar = P.scalar;
      const Mat* ms[3] = {&lay.m[0], &lay.m[1], &lay.m[2]};
      product(a, ms, nm, rows_of(0), tile_of(0));
    }
    const float* cs = hd == 512 ? c->gm_rope.as<float>() : c->rope.as<float>();
    const float* sn = cs + (size_t)c->ctxcap * (hd / 2);
    launch_pf_qkv(R.q, R.k, R.v, qn, kn, cs, sn, KCo, VCo, pos0, M, st, sib, hd, own, dpos);
    const float* ogs = nullptr;  // group sums of the staged attention rows (split path)
    bool oq = false;             // W4A8: the merge also quantised the rows for o
    if (split) pmark(c, PT_ATTN, 1, 0);  // the split-KV attention (E:1327 T_ATT)
    if (split && spd) {
      const int ty = hd == 512;
      oq = a8;
      if (hd == 512)
        launch_attn_geom_dev_hd(KCo, VCo, R.q, NQ * 512, geo + ty, M, nsplit, NQ, c->po5.as<float>(),
                                c->pm5.as<float>(), c->pl5.as<float>(), R.att, NQ * 512, st, attgs,
                                oq ? c->q8w.as<uint64_t>() : nullptr, oq ? c->q8s.as<float>() : nullptr);
      else
        launch_attn_geom_dev(KCo, VCo, R.q, NQ * HD, geo + ty, M, nsplit, c->po.as<float>(), c->pm.as<float>(),
                             c->pl.as<float>(), R.att, NQ * HD, st, NQ, attgs, oq ? c->q8w.as<uint64_t>() : nullptr,
                             oq ? c->q8s.as<float>() : nullptr);
      ogs = attgs;
    } else if (split) {
      AttnGeom ag{};
      ag.M = M;
      ag.kmax = pos0 + M - 1;
      ag.kmin = ag.kmax;
      ag.T = nsplit;
      for (int m = 0; m < M; ++m) {
        const int rp = m == sib ? pos0 + 1 : pos0 + m;
        ag.pos[m] = pos0 + m;
        ag.lo[m] = sliding ? std::max(0, rp - 511) : 0;
        ag.skip_lo[m] = m == sib ? pos0 + 1 : 1;
        ag.skip_hi[m] = m == sib ? pos0 + m - 1 : 0;
        ag.kmin = std::min(ag.kmin, ag.lo[m]);
      }
      if (hd == 512)
        (void)launch_attn_geom_hd(KCo, VCo, R.q, NQ * 512, ag, 512, c->po5.as<float>(), c->pm5.as<float>(),
                                  c->pl5.as<float>(), R.att, NQ * 512, attgs, st);
      else
        launch_attn_geom(KCo, VCo, R.q, NQ * HD, ag, c->po.as<float>(), c->pm.as<float>(), c->pl.as<float>(), R.att,
                         NQ * HD, st, NQ, attgs);
      ogs = attgs;
    } else {  // attn_tile (M >= 4 past 64 keys, no sibling) or run_mh
      launch_pf_attn(R.q, KCo, VCo, c->gm_s.as<float>(), R.att, PfGeom{M, pos0, M, sib}, 0, M, sliding, st, true, hd,
                     dpos, c->ctxcap);
    }
    if (split) pmark(c, PT_ATTN, 0, 0);
    {  // E:1356
      GemvTArgs a{};
      a.mat[0] = lay.m[3].tile();
      a.y[0] = R.o;
      a.ldy[0] = H;
      a.xs = reinterpret_cast<const float4*>(R.att);
      a.gs = ogs;
      if (oq) {
        a.xq = c->q8w.as<uint64_t>();
        a.xqs = c->q8s.as<float>();
      }
      a.K = NQ * hd;
      a.M = M;
      const Mat* ms[1] = {&lay.m[3]};
      product(a, ms, 1, rows_of(1), tile_of(1));
    }
    {  // E:1358-1371: the attention residual and pre-FF norm, then gate / up and gelu
      GemvTArgs a{};
      a.mat[0] = W4Tile{lay.m[4].tw.as<uint4>(), lay.m[4].ts.as<uint4>(), G.I};
      a.gateup = 1;
      a.y[0] = R.act;
      a.ldy[0] = G.I;
      a.nrm_mode = 1;
      a.nrm_o = R.o;
      a.nrm_xin = xa;
      a.nrm_xout = xb;
      a.nrm_w1 = post_attn;
      a.nrm_w2 = pre_ff;
      a.K = H;
      a.M = M;
      if (a8) {  // the gate and up matrices' own a8 tiles (their pairs meet in one block)
        a.mat[0] = a8t(lay.m[4]);
        a.mat[1] = a8t(lay.m[5]);
        if (a8_gateup_quantises(G.I)) {  // the activation quantised for down by the same blocks
          a.yq = c->q8w.as<uint64_t>();
          a.yqs = c->q8s.as<float>();
        }
        (void)launch_gemv_a8(a, st);
      } else {
        launch_gemv_t(a, st, rows_of(2), tile_of(2));
      }
    }
    bool down_done = false;  // E:1373
    if (a8) {
      GemvTArgs a{};
      a.mat[0] = a8t(lay.m[6]);
      a.y[0] = R.o;
      a.ldy[0] = H;
      a.xs = reinterpret_cast<const float4*>(R.act);
      if (a8_gateup_quantises(G.I)) {
        a.xq = c->q8w.as<uint64_t>();
        a.xqs = c->q8s.as<float>();
      }
      a.K = G.I;
      a.M = M;
      (void)launch_gemv_a8(a, st);
      down_done = true;
    } else if (lay.m[6].tw.p) {
      GemvTArgs a{};
      a.mat[0] = lay.m[6].tile();
      a.y[0] = R.o;
      a.ldy[0] = H;
      a.xs = reinterpret_cast<const float4*>(R.act);
      a.K = G.I;
      a.M = M;
      // the wide shape runs one activation row per block
      const bool wide = G.I > 6144;
      down_done = launch_gemv_t(a, st, wide ? 1 : rows_of(3), wide ? (M == 1 ? 32 : 64) : tile_of(3)) > 0;
    }
    if (!down_done) {
      GemvArgs a{};
      a.mat[0] = lay.m[6].dev();
      a.y[0] = R.o;
      a.ldy[0] = H;
      a.xs = reinterpret_cast<const float4*>(R.act);
      a.K = G.I;
      a.M = M;
      launch_gemv(a, EPI_STORE, st);
    }
    {  // E:1375-1385: the MLP residual, then the per-layer-input gate, gelu x the layer's input
      GemvTArgs a{};
      a.mat[0] = G.pg.tile();
      a.y[0] = R.g2;
      a.ldy[0] = GM_PD;
      a.nrm_mode = 3;
      a.nrm_o = R.o;
      a.nrm_xin = xb;
      a.nrm_xout = xc;
      a.nrm_w1 = post_ff;
      a.nrm_w2 = post_ff;  // (no second norm in this mode)
      a.epi_pli = R.pli + (size_t)l * GM_PD;
      a.epi_pli_ld = GM_PLN;
      a.K = H;
      a.M = M;
      const Mat* ms[1] = {&G.pg};
      product(a, ms, 1, 1, M == 1 ? 32 : 64);
    }
    {  // E:1386
      GemvTArgs a{};
      a.mat[0] = G.pp.tile();
      a.y[0] = R.o;
      a.ldy[0] = H;
      a.xs = reinterpret_cast<const float4*>(R.g2);
      a.K = GM_PD;
      a.M = M;
      const Mat* ms[1] = {&G.pp};
      product(a, ms, 1, 1, M == 1 ? 32 : 64);
    }
  }
  // E:1387-1404 and 1414-1417 of the last layer: its per-layer-input residual, scalar, final norm
  const auto& L = c->gm[GM_NL - 1];
  launch_pf_post_ff(R.o, xc, xb, L.nv.as<float>() + 4 * H, nullptr, c->fnorm.as<float>(), L.scalar, h, 0, M, st, hn);
}
}  // namespace

extern "C" {

int g4v_model_create_gemma(g4v_ctx* c, int V, const int* mlp, int ctxcap) {
  if (!c || !mlp) return G4V_E_ARG;
  ARGCHK(V > 0 && ctxcap > 8 && ctxcap <= 131072, "model_create_gemma: need V > 0 and 8 < ctxcap <= 131072");
  int Imax = 0;
  for (int l = 0; l < GM_NL; ++l) {
    ARGCHK(mlp[l] > 0 && mlp[l] % 256 == 0 && mlp[l] <= 16384, "model_create_gemma: MLP widths % 256 == 0, <= 16384");
    Imax = std::max(Imax, mlp[l]);
  }
  HIPCHK(hipSetDevice(c->device));
  int r = model_alloc(c, V, GM_NL, 256, ctxcap);
  if (r) return r;
  ALLOC(c->gm_geo, 2 * sizeof(AttnGeom));
  c->gemma = true;
  c->gm_Imax = Imax;
  c->gm_plready = false;
  size_t off = 0;
  for (int l = 0; l < GM_NL; ++l) {
    auto& G = c->gm[l];
    for (DBuf* b : {&G.pg.wr, &G.pg.s, &G.pg.tw, &G.pg.ts, &G.pg.a8w, &G.pg.a8s, &G.pp.wr, &G.pp.s, &G.pp.tw, &G.pp.ts,
                    &G.pp.a8w, &G.pp.a8s})
      b->reset();
    G.normed = false;
    G.scalar = 1.0f;
    G.hd = gm_hd(l);
    G.own = l < 15;
    G.I = mlp[l];
    ALLOC(G.nv, (size_t)(5 * H + 2 * G.hd) * 4);
    HIPCHK(hipMemsetAsync(G.nv.p, 0, G.nv.n, c->st));
    if (G.own) {
      c->gm_koff[l] = off;
      off += (size_t)c->kvcap * G.hd;
      c->gm_voff[l] = off;
      off += (size_t)c->kvcap * G.hd;
    }
  }
  ALLOC(c->gm_kv, off * 2);
  HIPCHK(hipMemsetAsync(c->gm_kv.p, 0, c->gm_kv.n, c->st));
  ALLOC(c->gm_ple, (size_t)V * GM_PLN * 2);
  HIPCHK(hipMemsetAsync(c->gm_ple.p, 0, c->gm_ple.n, c->st));
  ALLOC(c->gm_plnorm, GM_PD * 4);
  {  // E:1246-1247, the global type: theta 1e6 on the first quarter of the 256 frequencies
    std::vector<float> rt((size_t)2 * ctxcap * 256);
    for (int p = 0; p < ctxcap; ++p)
      for (int j = 0; j < 256; ++j) {
        const double inv = j < 64 ? 1.0 / std::pow(1e6, (2.0 * j) / 512) : 0.0;
        const double ang = p * inv;
        rt[(size_t)p * 256 + j] = (float)std::cos(ang);
        rt[(size_t)ctxcap * 256 + (size_t)p * 256 + j] = (float)std::sin(ang);
      }
    ALLOC(c->gm_rope, rt.size() * 4);
    HIPCHK(hipMemcpy(c->gm_rope.p, rt.data(), rt.size() * 4, hipMemcpyHostToDevice));
  }
  c->gm_cap = 0;
  c->gm_sfl = 0;
  r = gm_reserve(c, GM_ROWS, (size_t)pf_score_floats(GM_ROWS, ctxcap, 0));  // a prompt block / verify pass
  if (r) return r;
  ALLOC(c->po5, (size_t)MAXT * MAXM * NQ * 512 * 4);
  ALLOC(c->pm5, (size_t)MAXT * MAXM * NQ * 4);
  ALLOC(c->pl5, (size_t)MAXT * MAXM * NQ * 4);
  c->pf_rows = 0;  // the synthetic stack's prefill buffers are not sized for this layout
  HIPCHK(hipStreamSynchronize(c->st));
  c->model_ready = true;
  return 0;
}

int g4v_model_set_norms_gemma(g4v_ctx* c, int l, const float* const nv[7], float scalar) {
  if (!c || !nv) return G4V_E_ARG;
  ARGCHK(c->gemma && l >= 0 && l < GM_NL, "model_set_norms_gemma: no Gemma layout, or layer out of range");
  auto& G = c->gm[l];
  for (int t = 0; t < 7; ++t)
    ARGCHK(nv[t] != nullptr || (t == 6 && !G.own), "model_set_norms_gemma: null norm vector");
  HIPCHK(hipSetDevice(c->device));
  for (int t = 0; t < 7; ++t) {
    if (!nv[t]) continue;
    const size_t n = t < 5 ? H : G.hd, o = t < 5 ? (size_t)t * H : 5 * H + (size_t)(t - 5) * G.hd;
    HIPCHK(hipMemcpyAsync(G.nv.as<float>() + o, nv[t], n * 4, hipMemcpyHostToDevice, c->st));
  }
  HIPCHK(hipStreamSynchronize(c->st));
  if (G.scalar != scalar) drop_graphs(c);  // the layer scalar is baked into captured passes
  G.scalar = scalar;
  G.normed = true;
  return 0;
}

int g4v_model_set_ple(g4v_ctx* c, const uint8_t* w, const uint16_t* s, const float* plnorm) {
  if (!c || !w || !s || !plnorm) return G4V_E_ARG;
  ARGCHK(c->gemma, "model_set_ple: no Gemma layout (g4v_model_create_gemma first)");
  HIPCHK(hipSetDevice(c->device));
  drop_graphs(c);  // the projection's buffers are reallocated
  DBuf tmp;
  ALLOC(tmp, (size_t)GM_PLN * H / 2);
  HIPCHK(hipMemcpyAsync(tmp.p, w, (size_t)GM_PLN * H / 2, hipMemcpyHostToDevice, c->st));
  int r = upload_w4(c, c->gm_plproj, tmp.as<uint8_t>(), s, false, GM_PLN, H);
  if (r) return r;
  HIPCHK(hipMemcpyAsync(c->gm_plnorm.p, plnorm, GM_PD * 4, hipMemcpyHostToDevice, c->st));
  HIPCHK(hipStreamSynchronize(c->st));
  c->gm_plready = true;
  return 0;
}

int g4v_model_set_ple_rows(g4v_ctx* c, int tok0, int n, const uint16_t* rows) {
  if (!c || !rows) return G4V_E_ARG;
  ARGCHK(c->gemma && tok0 >= 0 && n >= 0 && (long long)tok0 + n <= c->V, "model_set_ple_rows: rows outside the table");
  HIPCHK(hipSetDevice(c->device));
  HIPCHK(hipMemcpy(c->gm_ple.as<uint16_t>() + (size_t)tok0 * GM_PLN, rows, (size_t)n * GM_PLN * 2,
                   hipMemcpyHostToDevice));
  return 0;
}

}  // extern "C"

extern "C" {

// a Gemma-4-E2B layout with weights generated on the device from `seed` (no checkpoint): the
// embedding f2bf(0.02 normal), int4 matrices with scales as g4v_model_synth draws them, norm
// vectors r16(0.5 + unif) (q / k norms r16(0.2 + 0.1 unif)), layer scalars 0.75, the per-layer
// embedding table f2bf(0.5 normal) for every token
extern "C" int g4v_model_synth_gemma(g4v_ctx* c, uint64_t seed, int V, const int* mlp, int ctxcap) {
  int r = g4v_model_create_gemma(c, V, mlp, ctxcap);
  if (r) return r;
  hipStream_t st = c->st;
  launch_gen_bf16_normal(c->E.as<uint16_t>(), (size_t)V * H, rng_stream(seed, 1), 0.02f, st);
  r = head_build_dev(c, V);
  if (r) return r;
  c->head_ready = true;
  size_t maxw = (size_t)GM_PLN * H;
  for (int l = 0; l < GM_NL; ++l)
    for (int j = 0; j < 9; ++j) {
      int N, K;
      gm_shape(c, l, j, &N, &K);
      maxw = std::max(maxw, (size_t)N * K);
    }
  DBuf tw, ts;
  ALLOC(tw, maxw / 2);
  ALLOC(ts, maxw / 16);
  auto gen_mat = [&](Mat& m, int N, int K, uint64_t tag, bool tiled = false) -> int {
    launch_gen_w4(tw.as<uint8_t>(), ts.as<uint16_t>(), (size_t)N * K / 2, (size_t)N * K / 32, rng_stream(seed, tag),
                  rng_stream(seed, tag + 500000), st);
    return upload_w4(c, m, tw.as<uint8_t>(), ts.as<uint16_t>(), true, N, K, tiled);
  };
  for (int l = 0; l < GM_NL; ++l) {
    auto& G = c->gm[l];
    for (int j = 0; j < 9; ++j) {
      if (!G.own && (j == 1 || j == 2)) continue;
      int N, K;
      gm_shape(c, l, j, &N, &K);
      if ((r = gen_mat(gm_mat(c, l, j), N, K, 1000 + 10 * (uint64_t)l + j, gm_tiled(j, K)))) return r;
    }
    if ((r = tile_gateup(c, *c->L[l]))) return r;
    std::vector<float> nv(5 * H + 2 * G.hd, 0.f);
    for (int t = 0; t < 7; ++t) {
      if (t == 6 && !G.own) continue;
      const int n = t < 5 ? H : G.hd, off = t < 5 ? t * H : 5 * H + (t - 5) * G.hd;
      const float base = t < 5 ? 0.5f : 0.2f, span = t < 5 ? 1.0f : 0.1f;
      const uint64_t sn = rng_stream(seed, 3000 + 10 * (uint64_t)l + t);
      for (int i = 0; i < n; ++i) nv[off + i] = r16(base + span * rng_unif(sn, i));
    }
    HIPCHK(hipMemcpy(G.nv.p, nv.data(), nv.size() * 4, hipMemcpyHostToDevice));
    G.scalar = 0.75f;
    G.normed = true;
  }
  if ((r = gen_mat(c->gm_plproj, GM_PLN, H, 900))) return r;
  std::vector<float> pn(GM_PD), fn(H);
  const uint64_t sp = rng_stream(seed, 901), sf = rng_stream(seed, 4000);
  for (int i = 0; i < GM_PD; ++i) pn[i] = r16(0.5f + rng_unif(sp, i));
  for (int i = 0; i < H; ++i) fn[i] = r16(0.5f + rng_unif(sf, i));
  HIPCHK(hipMemcpy(c->gm_plnorm.p, pn.data(), GM_PD * 4, hipMemcpyHostToDevice));
  HIPCHK(hipMemcpy(c->fnorm.p, fn.data(), H * 4, hipMemcpyHostToDevice));
  launch_gen_bf16_normal(c->gm_ple.as<uint16_t>(), (size_t)V * GM_PLN, rng_stream(seed, 902), 0.5f, st);
  HIPCHK(hipGetLastError());
  HIPCHK(hipStreamSynchronize(st));
  c->gm_plready = true;
  return 0;
}

static int gm_set_matrix(g4v_ctx* c, int l, int j, const uint8_t* w, const uint16_t* s) {
  ARGCHK(l >= 0 && l < GM_NL && j >= 0 && j < 9, "model_set_matrix: layer or matrix index out of range");
  ARGCHK(c->gm[l].own || (j != 1 && j != 2), "model_set_matrix: layers past 14 have no k / v projection (E:1251)");
  int N, K;
  gm_shape(c, l, j, &N, &K);
  DBuf tmp;
  ALLOC(tmp, (size_t)N * K / 2);
  HIPCHK(hipMemcpyAsync(tmp.p, w, (size_t)N * K / 2, hipMemcpyHostToDevice, c->st));
  int r = upload_w4(c, gm_mat(c, l, j), tmp.as<uint8_t>(), s, false, N, K, gm_tiled(j, K));
  if (r) return r;
  if ((j == 4 || j == 5) && (r = tile_gateup(c, *c->L[l]))) return r;
  HIPCHK(hipStreamSynchronize(c->st));
  return 0;
}

// the verify pass on the Gemma layout: a chain of up to 7 drafts or the sibling form (nb = 1,
// at most 4 rows); fwd as one block, then the head passes and acceptance of the verify pass
static int gm_verify(g4v_ctx* c, const int* toks, int na, int nb, int pos0, int nsplit, int b_ok,
                     g4v_verify_result* out, float* hidden) {
  std::string what;
  if (!c->model_ready || !gm_complete(c, &what)) {
    c->err = "verify_step: " + (c->model_ready ? what : std::string("no model"));
    return G4V_E_STATE;
  }
  const int M = 1 + na + nb;
  ARGCHK(toks && out && na >= 0 && nb >= 0 && na <= 7 && nb <= 1 && M <= MAXM && (nb == 0 || M <= 4),
         "verify_step: the Gemma layout takes a chain of up to 7 drafts or the sibling form");
  ARGCHK(nb == 0 || na >= 1, "verify_step: branch b needs a chain a");
  ARGCHK(pos0 >= 1 && pos0 + M <= c->ctxcap, "verify_step: positions beyond the cache");
  ARGCHK(nsplit >= 1 && nsplit <= MAXT, "verify_step: 1 <= nsplit <= 16");
  // only a pass of at most 4 rows past ATT_PAR takes the split-KV path (E:1305): the per-split
  // limit of the split buffer applies to it alone
  ARGCHK(!(M <= 4 && pos0 + M > 192) || (pos0 + M + nsplit - 1) / nsplit + 1 <= std::min(attn_pmax(), ATT_SPLIT_MAX - 1),
         "verify_step: context too long for nsplit");
  for (int i = 0; i < M; ++i) ARGCHK(toks[i] >= 0 && toks[i] < c->V, "verify_step: token id out of range");
  HIPCHK(hipSetDevice(c->device));
  hipStream_t st = c->st;
  StepDev& s = *c->step_host;
  std::memset(&s, 0, sizeof s);
  s.M = M;
  s.na = na;
  s.nb = nb;
  s.pos0 = pos0;
  s.b_ok = b_ok;
  for (int r = 0; r < M; ++r) {
    s.toks[r] = toks[r];
    s.rope[r] = r <= na ? pos0 + r : pos0 + 1;
    s.skip_lo[r] = r <= na ? 1 : pos0 + 1;
    s.skip_hi[r] = r <= na ? 0 : pos0 + na;
  }
  // The pass reads its tokens and positions from the step parameters on the device (copied in by
  // its first node from the pinned step block), so a shape is captured once as a graph (after one
  // eager run) and replayed at every position; the key holds what the launches bake in: rows,
  // branches, splits, the attention path (E:1305-1337) and the W4A8 mode.
  const int sib = nb == 1 ? na + 1 : -1;
  const bool i8p = c->dec_i8 && c->pf_i8 && M >= 2;  // G_I8_ACTIVE in the decode (E:1600), lin_multi's M >= 2 (E:311)
  const int path = (M <= 4 && pos0 + M > 192) ? 0 : 1;
  const long long key =
      (1LL << 62) | ((((((long long)M * 8 + na) * 8 + nb) * 32 + nsplit) * 2 + path) * 2 + (i8p ? 1 : 0));
  auto enqueue = [&]() {
    (void)hipMemcpyAsync(c->stepd.p, &s, sizeof s, hipMemcpyHostToDevice, st);
    const StepDev* sp = c->stepd.as<StepDev>();
    gm_verify_forward(c, M, pos0, nsplit, sib, c->h.as<float>(), c->hn.as<float>(), sp, i8p);
    VerifyResultDev* res = c->resd.as<VerifyResultDev>();
    head_run(head_args(c, c->hb1, c->h.as<float>(), c->hn.as<float>(), 1, nullptr), st);  // E:1453-1488
    launch_branch(sp, c->hb1.hs.best, c->h.as<float>(), c->hn.as<float>(), c->h2.as<float>(), c->hn2.as<float>(),
                  res, st);
    HeadRun h2 = head_args(c, c->hb2, c->h2.as<float>(), c->hn2.as<float>(), std::max(1, std::max(na, nb)),
                           &res->hcount);
    h2.pass2 = 1;
    head_run(h2, st);
    launch_accept(sp, c->hb1.hs.best, c->hb2.hs.best, c->hb1.hs.cnt, c->hb2.hs.cnt, res, nullptr, nullptr, 0, 0, st);
    for (int l = 0; l < 15; ++l)  // E:1651: the sibling's rows move into place in every owner cache
      launch_kv_compact_hd(sp, res, c->gm_kv.as<uint16_t>() + c->gm_koff[l], c->gm_kv.as<uint16_t>() + c->gm_voff[l],
                           c->gm[l].hd, st);
    (void)hipMemcpyAsync(c->res_host, c->resd.p, sizeof(VerifyResultDev), hipMemcpyDeviceToHost, st);
  };
  g4v_ctx::Graph* gr = nullptr;
  for (auto& g : c->graphs)
    if (g.key == key) gr = &g;
  const bool warm = std::find(c->warmed.begin(), c->warmed.end(), key) != c->warmed.end();
  if (gr) {
    HIPCHK(hipGraphLaunch(gr->exec, st));
  } else if (!c->use_graph || !warm) {  // the first pass of a shape (or graphs disabled) runs eagerly
    enqueue();
    HIPCHK(hipGetLastError());
    if (!warm) c->warmed.push_back(key);
  } else {
    g4v_ctx::Graph g;
    g.key = key;
    hipGraph_t graph;
    HIPCHK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    enqueue();
    HIPCHK(hipStreamEndCapture(st, &graph));
    const hipError_t ei = hipGraphInstantiate(&g.exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (ei != hipSuccess) {
      c->err = std::string("hipGraphInstantiate: ") + hipGetErrorString(ei);
      return G4V_E_HIP;
    }
    c->graphs.push_back(std::move(g));
    gr = &c->graphs.back();
    HIPCHK(hipGraphLaunch(gr->exec, st));
  }
  HIPCHK(hipStreamSynchronize(st));
  const VerifyResultDev& r = *c->res_host;
  // per-class timing (g4v_profile) of a pass launched eagerly; a captured pass's launches record
  // no events of their own here, so profiling these passes wants graphs off (g4v_set_graphs(0))
  if (c->prof_mask) {
    if (gr) {
      c->recs.clear();
      c->evused = 0;
    } else {
      prof_collect(c, r.fallback[0] != 0);
    }
  }
  out->nacc = r.nacc;
  out->branch = r.branch;
  out->ncommit = r.ncommit;
  for (int i = 0; i < 8; ++i) {
    out->commit[i] = r.commit[i];
    out->G[i] = r.G[i];
    out->fallback[i] = r.fallback[i];
    out->nsurv[i] = r.nsurv[i];
  }
  c->last_hrow = r.hrows[r.ncommit - 1];
  if (hidden)
    HIPCHK(hipMemcpy(hidden, c->h.as<float>() + (size_t)c->last_hrow * H, H * 4, hipMemcpyDeviceToHost));
  return 0;
}

// run_req's prompt loop (E:1594-1599) on the Gemma layout: blocks of pfb rows from pos0, the last
// block's last row to the head
static int gm_prefill(g4v_ctx* c, const int* toks, int n, int pos0, int pfb, int nsplit, int* G0, float* hidden) {
  std::string what;
  if (!c->model_ready || !gm_complete(c, &what)) {
    c->err = "prefill: " + (c->model_ready ? what : std::string("no model"));
    return G4V_E_STATE;
  }
  ARGCHK(toks && n >= 1 && pos0 >= 0 && (long long)pos0 + n <= c->ctxcap, "prefill: positions beyond the cache");
  ARGCHK(pfb >= 1 && pfb <= GM_ROWS, "prefill: 1 <= pfb <= 32 (the engine's row block, MM = 32)");
  ARGCHK(nsplit >= 1 && nsplit <= MAXT, "prefill: 1 <= nsplit <= 16");
  for (int i = 0; i < n; ++i) ARGCHK(toks[i] >= 0 && toks[i] < c->V, "prefill: token id outside the vocabulary");
  // blocks of 5 rows or more take attn_tile / run_mh only (E:1305, 1328): every block but a last
  // one that is short (split-KV past ATT_PAR) or a single row (exact float, E:311) runs in one
  // pass; smaller blocks run one by one
  const int Ml = n - (n - 1) / pfb * pfb, p0l = pos0 + n - Ml;
  const bool tail = (Ml <= 4 && p0l + Ml > 192) || Ml == 1;
  const int nA = pfb >= 5 ? (tail ? n - Ml : n) : 0;
  // the per-split limit of the split buffer binds only the blocks that take the split-KV path
  // (at most 4 rows past ATT_PAR, E:1305), the last of which ends at pos0 + n
  const bool split_blocks = pfb >= 5 ? (tail && Ml <= 4 && p0l + Ml > 192) : pos0 + n > 192;
  ARGCHK(!split_blocks || (pos0 + n + nsplit - 1) / nsplit + 1 <= std::min(attn_pmax(), ATT_SPLIT_MAX - 1),
         "prefill: more positions per split than the split buffer holds");
  HIPCHK(hipSetDevice(c->device));
  if (nA > 0) {
    int r = gm_reserve(c, nA, (size_t)pf_score_floats(nA, pos0, 0));
    if (r) return r;
    HIPCHK(hipMemcpyAsync(c->gm_tok.p, toks, (size_t)nA * 4, hipMemcpyHostToDevice, c->st));
    const PfGeom g{n, pos0, pfb, -1};
    gm_forward(c, nA, pos0, nsplit, -1, nA == n ? nA - 1 : -1, c->pf_i8, c->h.as<float>(), c->hn.as<float>(), &g);
  }
  for (int b = nA; b < n; b += pfb) {
    const int M = std::min(pfb, n - b);
    const bool last = b + M == n;
    HIPCHK(hipMemcpyAsync(c->gm_tok.p, toks + b, (size_t)M * 4, hipMemcpyHostToDevice, c->st));
    gm_forward(c, M, pos0 + b, nsplit, -1, last ? M - 1 : -1, c->pf_i8, c->h.as<float>(), c->hn.as<float>());
  }
  HIPCHK(hipGetLastError());
  std::vector<float> h(H);
  HIPCHK(hipMemcpyAsync(h.data(), c->h.p, H * 4, hipMemcpyDeviceToHost, c->st));
  HIPCHK(hipStreamSynchronize(c->st));
  c->last_hrow = 0;  // the prompt's last row: the state a drafter chain would start from
  if (hidden) std::memcpy(hidden, h.data(), H * 4);
  if (G0) {
    int ns = 0, fb = 0;
    const int rr = g4v_head_argmax(c, h.data(), 1, G0, &ns, &fb);
    c->pf_nsurv = ns;
    c->pf_fallback = fb;
    return rr;
  }
  return 0;
}

extern "C" int g4v_prefill(g4v_ctx* c, const int* toks, int n, int pos0, int pfb, int nsplit, int* G0,
                           float* hidden) {
  if (!c) return G4V_E_ARG;
  if (c->gemma) return gm_prefill(c, toks, n, pos0, pfb, nsplit, G0, hidden);
  std::string what;
  if (!c->model_ready || !model_complete(c, &what)) {
    c->err = "prefill: " + (c->model_ready ? what : std::string("no model"));
    return G4V_E_STATE;
  }
  ARGCHK(toks && n >= 1 && pos0 >= 0, "prefill: need tokens, n >= 1, pos0 >= 0");
  ARGCHK((long long)pos0 + n <= c->ctxcap, "prefill: pos0 + n beyond the context capacity");
  ARGCHK(pfb >= 1 && pfb <= 32, "prefill: 1 <= pfb <= 32 (the engine's row block, MM = 32)");
  // a block before the last one of at most 4 rows past ATT_PAR takes the split-KV path (E:1305),
  // of one row the exact-float products (E:311): only the last block is run that way here
  ARGCHK(pfb >= 5 || (n - 1) / pfb == 0 || pos0 + (n - 1) / pfb * pfb <= 192,
         "prefill: pfb < 5 with blocks before the last past position 192 (split-KV blocks) is not supported");
  ARGCHK(pfb >= 2 || n == 1 || !c->pf_i8,
         "prefill: pfb 1 (one exact-float row per block) with W4A8 prefill is not supported for n > 1");
  ARGCHK(nsplit >= 1 && nsplit <= MAXT, "prefill: 1 <= nsplit <= 16");
  for (int i = 0; i < n; ++i) ARGCHK(toks[i] >= 0 && toks[i] < c->V, "prefill: token id outside the vocabulary");
  HIPCHK(hipSetDevice(c->device));
  // the last block; a short one past ATT_PAR = 192 (E:1214) takes the split-KV path, a 1-row one
  // the exact-float GEMV (lin_multi's M >= 2 rule): both run as a segment of their own
  const int Ml = n - (n - 1) / pfb * pfb, p0l = pos0 + n - Ml;
  const bool tsplit = Ml <= 4 && p0l + Ml > 192, tail = tsplit || Ml == 1;
  const int nA = tail ? n - Ml : n;
  if (tsplit)
    ARGCHK((Ml + p0l + nsplit - 1) / nsplit <= attn_pmax(), "prefill: more positions per split than the split buffer holds");
  size_t sfl = 0;
  for (int l = 0; l < c->NL; ++l) {
    sfl = std::max(sfl, (size_t)pf_score_floats(nA, pos0, c->L[l]->sliding));
    if (tail && !tsplit) sfl = std::max(sfl, (size_t)pf_score_floats(Ml, p0l, c->L[l]->sliding));
  }
  int r = pf_alloc(c, n, sfl);
  if (r) return r;
  HIPCHK(hipMemcpyAsync(c->pftok.p, toks, (size_t)n * 4, hipMemcpyHostToDevice, c->st));
  const PfGeom g{n, pos0, pfb, -1};
  if (nA > 0) pf_segment(c, g, 0, nA, c->pf_i8, false, nsplit, tail ? -1 : nA - 1);
  if (tail) pf_segment(c, g, nA, Ml, c->pf_i8 && Ml >= 2, tsplit, nsplit, Ml - 1);
  HIPCHK(hipGetLastError());
  std::vector<float> h(H);
  HIPCHK(hipMemcpyAsync(h.data(), c->pfh.p, H * 4, hipMemcpyDeviceToHost, c->st));
  HIPCHK(hipStreamSynchronize(c->st));
  if (hidden) std::memcpy(hidden, h.data(), H * 4);
  if (G0) {
    int ns = 0, fb = 0;
    r = g4v_head_argmax(c, h.data(), 1, G0, &ns, &fb);
    if (r) return r;
    c->pf_nsurv = ns;
    c->pf_fallback = fb;
  }
  return 0;
}


// ---------------------------------------------------------------------------------------
// MTP drafter
// ---------------------------------------------------------------------------------------
namespace {
constexpr int DR_H = 256, DR_Q = 4, DR_F = 2048, DR_NC = 32 * 128, DR_HDMAX = 512;
// drafter norms on the device: [4 layers][5: in_ln, post_attn, pre_ff, post_ff, q_norm][512],
// then the final norm [256]
constexpr int DR_NSTRIDE = 512, DR_NORM_FLOATS = 20 * DR_NSTRIDE + DR_H;
// scratch layout (floats / ints) of a drafter chain
constexpr int DR_IN_WORDS = 4 + H, DR_OUT_WORDS = 24 + H;
struct DrScratch {
  float *dx[2], *yo, *ydown, *dq, *dopt, *act, *dh, *bout[2], *hin, *dscore, *cscore, *gap;
  int *top, *tok, *sec, *din;
  AttnGeom* geo;  // [2 * 8]
};
DrScratch dr_scratch(g4v_ctx* c) {
  float* f = c->dr_s.as<float>();
  DrScratch d;
  d.dx[0] = f;
  d.dx[1] = d.dx[0] + DR_H;
  d.yo = d.dx[1] + DR_H;
  d.ydown = d.yo + DR_H;
  d.dq = d.ydown + DR_H;
  d.dopt = d.dq + DR_Q * DR_HDMAX;
  d.act = d.dopt + DR_Q * DR_HDMAX;
  d.dh = d.act + DR_F;
  d.bout[0] = d.dh + DR_H;
  d.bout[1] = d.bout[0] + H;
  d.hin = d.bout[1] + H;
  d.dscore = d.hin + H;
  d.cscore = d.dscore + 4096;
  d.gap = d.cscore + DR_NC;
  int* ip = reinterpret_cast<int*>(d.gap + 16);
  d.top = ip;
  d.tok = d.top + 32;
  d.sec = d.tok + 16;
  d.din = d.sec + 16;
  d.geo = reinterpret_cast<AttnGeom*>(d.din + DR_IN_WORDS);
  return d;
}
constexpr size_t DR_SCRATCH_BYTES = (size_t)(5 * DR_H + 2 * DR_Q * DR_HDMAX + DR_F + 3 * H + 4096 + DR_NC + 16) * 4 +
                                    (size_t)(32 + 16 + 16 + DR_IN_WORDS) * 4 + 16 * sizeof(AttnGeom);
}  // namespace

extern "C" int g4v_drafter_synth(g4v_ctx* c, uint64_t seed) {
  if (!c) return G4V_E_ARG;
  if (!c->model_ready) {
    c->err = "drafter_synth: no model";
    return G4V_E_STATE;
  }
  ARGCHK(c->V % 2048 == 0 && c->V / 128 >= 32 && c->V / 128 <= 4096,
         "drafter_synth: the vocabulary must be 128 x C tokens with 32 <= C <= 4096 centroids, C % 16 == 0");
  ARGCHK(c->NL >= 15, "drafter_synth: the drafter reads the KV cache of target layers 13 and 14");
  ARGCHK(!c->gemma, "drafter_synth: the Gemma layout's layer 14 has head dim 512: load a drafter checkpoint "
                    "(g4v_drafter_load)");
  HIPCHK(hipSetDevice(c->device));
  drop_graphs(c);  // captured chains hold the drafter buffers
  for (int l = 0; l < 4; ++l) {
    c->dr_hd[l] = HD;
    c->dr_scalar[l] = 0.75f;
  }
  hipStream_t st = c->st;
  const int V = c->V, C = V / 128;
  if (!c->dr_in_host) HIPCHK(hipHostMalloc((void**)&c->dr_in_host, DR_IN_WORDS * 4, hipHostMallocDefault));
  if (!c->dr_out_host) HIPCHK(hipHostMalloc((void**)&c->dr_out_host, DR_OUT_WORDS * 4, hipHostMallocDefault));
  auto gen = [&](DBuf& b, size_t n, uint64_t tag, float scale) -> int {
    ALLOC(b, n * 2);
    launch_gen_bf16_normal(b.as<uint16_t>(), n, rng_stream(seed, tag), scale, st);
    return 0;
  };
  int r;
  if ((r = gen(c->dr_pre, (size_t)DR_H * 2 * H, 5000, 0.02f))) return r;
  for (int l = 0; l < 4; ++l) {
    if ((r = gen(c->dr_q[l], (size_t)DR_Q * DR_H * DR_H, 5100 + 10 * l, 0.06f)) ||
        (r = gen(c->dr_o[l], (size_t)DR_H * DR_Q * DR_H, 5101 + 10 * l, 0.03f)) ||
        (r = gen(c->dr_g[l], (size_t)DR_F * DR_H, 5102 + 10 * l, 0.06f)) ||
        (r = gen(c->dr_u[l], (size_t)DR_F * DR_H, 5103 + 10 * l, 0.06f)) ||
        (r = gen(c->dr_d[l], (size_t)DR_H * DR_F, 5104 + 10 * l, 0.02f)))
      return r;
  }
  if ((r = gen(c->dr_post, (size_t)H * DR_H, 5300, 0.06f)) || (r = gen(c->dr_cent, (size_t)C * DR_H, 5301, 0.06f)) ||
      (r = gen(c->dr_emb, (size_t)V * DR_H, 5303, 0.06f)))
    return r;
  // norms (in_ln, post_attn, pre_ff, post_ff, q_norm per layer) then the final norm
  std::vector<float> nv(DR_NORM_FLOATS, 0.f);
  for (int l = 0; l < 4; ++l)
    for (int t = 0; t < 5; ++t) {
      const uint64_t sn = rng_stream(seed, 5200 + 10 * (uint64_t)l + t);
      const float base = t < 4 ? 0.5f : 0.2f, span = t < 4 ? 1.0f : 0.1f;
      for (int i = 0; i < DR_H; ++i) nv[(l * 5 + t) * DR_NSTRIDE + i] = r16(base + span * rng_unif(sn, i));
    }
  {
    const uint64_t sn = rng_stream(seed, 5302);
    for (int i = 0; i < DR_H; ++i) nv[20 * DR_NSTRIDE + i] = r16(0.5f + rng_unif(sn, i));
  }
  std::vector<int> order(V);
  for (int i = 0; i < V; ++i) order[i] = i;
  const uint64_t so = rng_stream(seed, 5304);
  for (int i = V - 1; i >= 1; --i) std::swap(order[i], order[(int)(rng_hash(so, (uint64_t)i) % (uint64_t)(i + 1))]);
  ALLOC(c->dr_norms, nv.size() * 4);
  ALLOC(c->dr_order, (size_t)V * 4);
  ALLOC(c->dr_s, DR_SCRATCH_BYTES);
  HIPCHK(hipMemcpyAsync(c->dr_norms.p, nv.data(), nv.size() * 4, hipMemcpyHostToDevice, st));
  HIPCHK(hipMemcpyAsync(c->dr_order.p, order.data(), (size_t)V * 4, hipMemcpyHostToDevice, st));
  HIPCHK(hipGetLastError());
  HIPCHK(hipStreamSynchronize(st));
  c->dr_C = C;
  c->dr_ready = true;
  return 0;
}

// E:1519-1528: a drafter checkpoint's tensors onto the device
extern "C" int g4v_drafter_load(g4v_ctx* c, const g4v_drafter_tensors* t) {
  if (!c || !t) return G4V_E_ARG;
  if (!c->model_ready) {
    c->err = "drafter_load: no model";
    return G4V_E_STATE;
  }
  ARGCHK(c->NL >= 15, "drafter_load: the drafter reads the KV cache of target layers 13 and 14");
  const int C = t->C, V = c->V;
  ARGCHK(C >= 32 && C <= 4096 && C % 16 == 0 && (long long)C * 128 == V,
         "drafter_load: the vocabulary must be 128 x C tokens with 32 <= C <= 4096 centroids, C % 16 == 0");
  const int hd14 = c->gemma ? c->gm[14].hd : HD;
  for (int l = 0; l < 4; ++l)
    ARGCHK(t->hd[l] == (l < 3 ? HD : hd14),
           "drafter_load: layers 0..2 have head dim 256, layer 3 that of the target's layer 14 (E:1525)");
  ARGCHK(t->pre && t->post && t->cent && t->emb && t->norm && t->order, "drafter_load: null tensor");
  for (int l = 0; l < 4; ++l) {
    ARGCHK(t->q[l] && t->o[l] && t->gate[l] && t->up[l] && t->down[l], "drafter_load: null tensor");
    for (int k = 0; k < 5; ++k) ARGCHK(t->nv[l][k], "drafter_load: null norm");
  }
  for (long long i = 0; i < V; ++i)
    ARGCHK(t->order[i] >= 0 && t->order[i] < V, "drafter_load: token ordering outside the vocabulary");
  HIPCHK(hipSetDevice(c->device));
  drop_graphs(c);  // captured chains hold the drafter buffers
  hipStream_t st = c->st;
  if (!c->dr_in_host) HIPCHK(hipHostMalloc((void**)&c->dr_in_host, DR_IN_WORDS * 4, hipHostMallocDefault));
  if (!c->dr_out_host) HIPCHK(hipHostMalloc((void**)&c->dr_out_host, DR_OUT_WORDS * 4, hipHostMallocDefault));
  auto put = [&](DBuf& b, const uint16_t* src, size_t n) -> int {
    ALLOC(b, n * 2);
    HIPCHK(hipMemcpyAsync(b.p, src, n * 2, hipMemcpyHostToDevice, st));
    return 0;
  };
  int r;
  if ((r = put(c->dr_pre, t->pre, (size_t)DR_H * 2 * H)) || (r = put(c->dr_post, t->post, (size_t)H * DR_H)) ||
      (r = put(c->dr_cent, t->cent, (size_t)C * DR_H)) || (r = put(c->dr_emb, t->emb, (size_t)V * DR_H)))
    return r;
  auto bf = [](uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
  };
  std::vector<float> nv(DR_NORM_FLOATS, 0.f);
  for (int l = 0; l < 4; ++l) {
    const int hd = t->hd[l];
    if ((r = put(c->dr_q[l], t->q[l], (size_t)DR_Q * hd * DR_H)) || (r = put(c->dr_o[l], t->o[l], (size_t)DR_H * DR_Q * hd)) ||
        (r = put(c->dr_g[l], t->gate[l], (size_t)DR_F * DR_H)) || (r = put(c->dr_u[l], t->up[l], (size_t)DR_F * DR_H)) ||
        (r = put(c->dr_d[l], t->down[l], (size_t)DR_H * DR_F)))
      return r;
    for (int k = 0; k < 5; ++k)
      for (int i = 0; i < (k < 4 ? DR_H : hd); ++i) nv[(l * 5 + k) * DR_NSTRIDE + i] = bf(t->nv[l][k][i]);
    c->dr_hd[l] = hd;
    c->dr_scalar[l] = bf(t->scalar[l]);
  }
  for (int i = 0; i < DR_H; ++i) nv[20 * DR_NSTRIDE + i] = bf(t->norm[i]);
  std::vector<int> order(V);
  for (int i = 0; i < V; ++i) order[i] = (int)t->order[i];
  ALLOC(c->dr_norms, nv.size() * 4);
  ALLOC(c->dr_order, (size_t)V * 4);
  ALLOC(c->dr_s, DR_SCRATCH_BYTES);
  HIPCHK(hipMemcpyAsync(c->dr_norms.p, nv.data(), nv.size() * 4, hipMemcpyHostToDevice, st));
  HIPCHK(hipMemcpyAsync(c->dr_order.p, order.data(), (size_t)V * 4, hipMemcpyHostToDevice, st));
  HIPCHK(hipStreamSynchronize(st));
  c->dr_C = C;
  c->dr_ready = true;
  return 0;
}

// the kernels of a k-step chain with nsplit attention splits; inputs from the pinned input
// block, outputs to the pinned output block (both copies are part of the sequence, so that a
// captured chain replays them)
static void enqueue_draft(g4v_ctx* c, int k, int nsplit) {
  hipStream_t st = c->st;
  const DrScratch d = dr_scratch(c);
  const float* nv = c->dr_norms.as<float>();
  auto nrm = [&](int l, int t) { return nv + (l * 5 + t) * DR_NSTRIDE; };
  (void)hipMemcpyAsync(d.din, c->dr_in_host, DR_IN_WORDS * 4, hipMemcpyHostToDevice, st);
  launch_dr_setup(d.din, c->h.as<float>(), d.hin, d.tok, d.geo, k, nsplit, st);
  for (int j = 0; j < k; ++j) {  // E:1631-1633: step j at position P + 1 + j, keys up to P
    const float* hj = j == 0 ? d.hin : d.bout[(j - 1) & 1];
    float* dxc = d.dx[0];  // the residual ping-pongs between d.dx[0] and d.dx[1]
    auto next_dx = [&]() { return dxc == d.dx[0] ? d.dx[1] : d.dx[0]; };
    {
      B16Launch L;
      L.W = c->dr_pre.as<uint16_t>(), L.N = DR_H, L.K = 2 * H, L.x = hj, L.y = dxc, L.pro = 3, L.epi = 1;
      L.E = c->E.as<uint16_t>(), L.tok = d.tok + j;
      launch_b16(L, st);
    }
    for (int l = 0; l < 4; ++l) {
      const bool sliding = l < 3;
      const int ty = sliding ? 0 : 1, ol = sliding ? 13 : 14, hd = c->dr_hd[l];  // E:1540
      // the target's RoPE table of the layer type ([ctxcap][hd / 2] cos, then sin) and cache of
      // layer 13 / 14: the synthetic stack's, or the Gemma layout's owner caches
      const float* cs = c->gemma && ty ? c->gm_rope.as<float>()
                                       : c->rope.as<float>() + (size_t)(2 * ty) * c->ctxcap * (HD / 2);
      const float* sn = cs + (size_t)c->ctxcap * (hd / 2);
      const uint16_t* Kl = c->gemma ? c->gm_kv.as<uint16_t>() + c->gm_koff[ol]
                                    : c->KC.as<uint16_t>() + (size_t)ol * c->kvcap * HD;
      const uint16_t* Vl = c->gemma ? c->gm_kv.as<uint16_t>() + c->gm_voff[ol]
                                    : c->VC.as<uint16_t>() + (size_t)ol * c->kvcap * HD;
      {  // q (E:1541), with the previous layer's post-FFN block in front (E:1548-1550)
        B16Launch L;
        L.W = c->dr_q[l].as<uint16_t>(), L.N = DR_Q * hd, L.K = DR_H, L.x = dxc, L.y = d.dq, L.nw = nrm(l, 0);
        if (l == 0) {
          L.pro = 1;
        } else {
          L.pro = 5, L.yin = d.ydown, L.w1 = nrm(l - 1, 3), L.scalar = c->dr_scalar[l - 1], L.dxout = next_dx();
          dxc = L.dxout;
        }
        launch_b16(L, st);
      }
      launch_dr_qnorm(d.dq, nrm(l, 4), cs, sn, d.din + 1, j, hd, st);
      if (hd == 512)
        launch_attn_geom_dev_hd(Kl, Vl, d.dq, DR_Q * hd, d.geo + 2 * j + ty, 1, nsplit, DR_Q, c->po5.as<float>(),
                                c->pm5.as<float>(), c->pl5.as<float>(), d.dopt, DR_Q * hd, st);
      else
        launch_attn_geom_dev(Kl, Vl, d.dq, DR_Q * hd, d.geo + 2 * j + ty, 1, nsplit, c->po.as<float>(),
                             c->pm.as<float>(), c->pl.as<float>(), d.dopt, DR_Q * hd, st, DR_Q);
      {  // o (E:1545)
        B16Launch L;
        L.W = c->dr_o[l].as<uint16_t>(), L.N = DR_H, L.K = DR_Q * hd, L.x = d.dopt, L.y = d.yo;
        launch_b16(L, st);
      }
      {  // gate / up + activation (E:1547), with the post-attention block in front (E:1545-1546)
        B16Launch L;
        L.W = c->dr_g[l].as<uint16_t>(), L.W2 = c->dr_u[l].as<uint16_t>(), L.N = DR_F, L.K = DR_H, L.x = dxc;
        L.y = d.act, L.pro = 4, L.epi = 2, L.yin = d.yo, L.w1 = nrm(l, 1), L.nw = nrm(l, 2), L.dxout = next_dx();
        dxc = L.dxout;
        launch_b16(L, st);
      }
      {  // down (E:1548)
        B16Launch L;
        L.W = c->dr_d[l].as<uint16_t>(), L.N = DR_H, L.K = DR_F, L.x = d.act, L.y = d.ydown;
        launch_b16(L, st);
      }
    }
    {  // the last post-FFN block, the final norm (E:1551), post-projection and centroid scores
      B16Launch L;
      L.W = c->dr_post.as<uint16_t>(), L.N = H, L.K = DR_H, L.x = dxc, L.y = d.bout[j & 1], L.pro = 6, L.epi = 1;
      L.yin = d.ydown, L.w1 = nrm(3, 3), L.scalar = c->dr_scalar[3], L.nw = nrm(4, 0), L.xout = d.dh;
      launch_b16(L, st);
      L.W = c->dr_cent.as<uint16_t>(), L.N = c->dr_C, L.y = d.dscore, L.epi = 0, L.xout = nullptr;
      launch_b16(L, st);
    }
    launch_dr_rank(d.dscore, c->dr_C, d.top, st);
    {  // the 32 x 128 candidates against dh (E:1556-1557)
      B16Launch L;
      L.W = c->dr_emb.as<uint16_t>(), L.N = DR_NC, L.K = DR_H, L.x = d.dh, L.y = d.cscore;
      L.top = d.top, L.order = c->dr_order.as<int>();
      launch_b16(L, st);
    }
    launch_dr_best(d.cscore, d.top, c->dr_order.as<int>(), DR_NC, d.tok + j + 1, d.sec + j, d.gap + j, st);
  }
  int* o = c->dr_out_host;
  (void)hipMemcpyAsync(o, d.tok + 1, (size_t)k * 4, hipMemcpyDeviceToHost, st);
  (void)hipMemcpyAsync(o + 8, d.sec, (size_t)k * 4, hipMemcpyDeviceToHost, st);
  (void)hipMemcpyAsync(o + 16, d.gap, (size_t)k * 4, hipMemcpyDeviceToHost, st);
  (void)hipMemcpyAsync(o + 24, d.bout[(k - 1) & 1], H * 4, hipMemcpyDeviceToHost, st);
}

extern "C" int g4v_draft_mtp(g4v_ctx* c, int tok, const float* h, int P, int k, int nsplit, int* drafts, int* sec,
                             float* gap, float* hidden) {
  if (!c) return G4V_E_ARG;
  if (!c->dr_ready) {
    c->err = "draft_mtp: no drafter (g4v_drafter_synth first)";
    return G4V_E_STATE;
  }
  ARGCHK(drafts && k >= 1 && k <= 8 && P >= 0 && P + k < c->ctxcap, "draft_mtp: 1 <= k <= 8, P + k < ctxcap");
  ARGCHK(tok >= 0 && tok < c->V, "draft_mtp: token outside the vocabulary");
  ARGCHK(nsplit >= 1 && nsplit <= MAXT && (P + 1 + nsplit - 1) / nsplit <= attn_pmax() &&
             (P + 1 + nsplit - 1) / nsplit + 1 <= ATT_SPLIT_MAX,
         "draft_mtp: 1 <= nsplit <= 16 and no more positions per split than the split buffer holds");
  if (!h && c->last_hrow < 0) {
    c->err = "draft_mtp: no hidden state given and no verify step ran";
    return G4V_E_STATE;
  }
  HIPCHK(hipSetDevice(c->device));
  int* in = c->dr_in_host;
  in[0] = tok;
  in[1] = P;
  in[2] = h ? -1 : c->last_hrow;
  in[3] = c->dr_same ? 1 : 0;
  if (h) std::memcpy(in + 4, h, H * 4);
  // captured once per (k, splits) after one eager run, like the verify pass; keys below zero
  const long long key = -1 - ((long long)k * 32 + nsplit);
  g4v_ctx::Graph* gr = nullptr;
  for (auto& g : c->graphs)
    if (g.key == key) gr = &g;
  const bool warm = std::find(c->warmed.begin(), c->warmed.end(), key) != c->warmed.end();
  if (gr) {
    HIPCHK(hipGraphLaunch(gr->exec, c->st));
  } else if (!c->use_graph || !warm) {
    enqueue_draft(c, k, nsplit);
    HIPCHK(hipGetLastError());
    if (!warm) c->warmed.push_back(key);
  } else {
    g4v_ctx::Graph g;
    g.key = key;
    hipGraph_t graph;
    HIPCHK(hipStreamBeginCapture(c->st, hipStreamCaptureModeThreadLocal));
    enqueue_draft(c, k, nsplit);
    HIPCHK(hipStreamEndCapture(c->st, &graph));
    const hipError_t ei = hipGraphInstantiate(&g.exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (ei != hipSuccess) {
      c->err = std::string("hipGraphInstantiate: ") + hipGetErrorString(ei);
      return G4V_E_HIP;
    }
    c->graphs.push_back(std::move(g));
    HIPCHK(hipGraphLaunch(c->graphs.back().exec, c->st));
  }
  HIPCHK(hipStreamSynchronize(c->st));
  const int* o = c->dr_out_host;
  for (int j = 0; j < k; ++j) drafts[j] = o[j];
  if (sec)
    for (int j = 0; j < k; ++j) sec[j] = o[8 + j];
  if (gap) std::memcpy(gap, o + 16, (size_t)k * 4);
  if (hidden) std::memcpy(hidden, o + 24, H * 4);
  return 0;
}


// ---------------------------------------------------------------------------------------
// prefix cache (run_req, E:1568-1593)
// ---------------------------------------------------------------------------------------
extern "C" int g4v_slots_init(g4v_ctx* c, int nslot, int min_reuse) {
  if (!c) return G4V_E_ARG;
  if (!c->model_ready) {
    c->err = "slots_init: no model";
    return G4V_E_STATE;
  }
  ARGCHK(nslot >= 1 && nslot <= 64, "slots_init: 1 <= nslot <= 64");
  HIPCHK(hipSetDevice(c->device));
  c->slots.clear();
  for (int i = 0; i + 1 < nslot; ++i) {
    auto sl = std::make_unique<g4v_ctx::Slot>();
    if (c->gemma) {  // the owner caches of the Gemma layout: one buffer
      ALLOC(sl->KC, c->gm_kv.n);
    } else {
      ALLOC(sl->KC, c->KC.n);
      ALLOC(sl->VC, c->VC.n);
    }
    c->slots.push_back(std::move(sl));
  }
  c->act_keys.clear();
  c->act_kv_len = 0;
  c->min_reuse = min_reuse;
  c->act_stamp = c->clock_tick = 0;
  return 0;
}

// the active KV and stored slot s exchange places (E:1576 swap_with): contents are swapped on the
// device, so captured passes keep pointing at the active cache
static int slot_swap(g4v_ctx* c, g4v_ctx::Slot& sl) {
  if (c->gemma) {
    launch_swap16(c->gm_kv.p, sl.KC.p, c->gm_kv.n, c->st);
  } else {
    launch_swap16(c->KC.p, sl.KC.p, c->KC.n, c->st);
    launch_swap16(c->VC.p, sl.VC.p, c->VC.n, c->st);
  }
  HIPCHK(hipGetLastError());
  std::swap(c->act_keys, sl.keys);
  std::swap(c->act_kv_len, sl.kv_len);
  std::swap(c->act_stamp, sl.stamp);
  return 0;
}

extern "C" int g4v_slot_begin(g4v_ctx* c, const int* toks, int n, int* start, int* slot_used) {
  if (!c) return G4V_E_ARG;
  if (!c->model_ready) {
    c->err = "slot_begin: no model";
    return G4V_E_STATE;
  }
  ARGCHK(toks && n >= 1 && start, "slot_begin: need n >= 1 tokens");
  HIPCHK(hipSetDevice(c->device));
  auto lcp_of = [&](const std::vector<int>& k, int klen) {  // E:1585
    int m = 0;
    while (m < klen && m < n && k[m] == toks[m]) ++m;
    return m;
  };
  int common = lcp_of(c->act_keys, c->act_kv_len), used = 0;
  ++c->clock_tick;
  if (!c->slots.empty()) {  // E:1587-1592
    int best = -1, bc = common;
    for (int i = 0; i < (int)c->slots.size(); ++i) {
      const int m = lcp_of(c->slots[i]->keys, c->slots[i]->kv_len);
      if (m > bc) {
        bc = m;
        best = i;
      }
    }
    if (best >= 0) {  // a stored conversation shares more: switch to it, park the active one there
      c->act_stamp = c->clock_tick;
      int r = slot_swap(c, *c->slots[best]);
      if (r) return r;
      used = best + 1;
      common = bc;
    } else if (bc < c->min_reuse) {  // nothing worth reusing: the LRU slot takes the active one
      int v = 0;
      for (int i = 1; i < (int)c->slots.size(); ++i)
        if (c->slots[i]->stamp < c->slots[v]->stamp) v = i;
      c->act_stamp = c->clock_tick;
      int r = slot_swap(c, *c->slots[v]);
      if (r) return r;
      c->act_kv_len = 0;
      c->act_keys.clear();
      common = 0;
      used = v + 1;
    }
    c->act_stamp = c->clock_tick;
  }
  *start = std::min(common, n - 1);  // E:1594: the last prompt token always runs again
  if (slot_used) *slot_used = used;
  HIPCHK(hipStreamSynchronize(c->st));
  return 0;
}

extern "C" int g4v_slot_end(g4v_ctx* c, const int* toks, int n, const int* gen, int ngen, int P) {
  if (!c) return G4V_E_ARG;
  ARGCHK(toks && n >= 1 && ngen >= 0 && (ngen == 0 || gen) && P >= n - 1, "slot_end: bad request record");
  // E:1671: the KV holds the prompt, then the generated tokens up to position P
  c->act_keys.assign(toks, toks + n);
  for (int i = 0; i <= P - n && i < ngen; ++i) c->act_keys.push_back(gen[i]);
  c->act_kv_len = std::min<int>(P + 1, (int)c->act_keys.size());
  return 0;
}

// history capacity for `need` tokens; keeps the first `keep` tokens
static int hist_reserve(g4v_ctx* c, int need, int keep) {
  if (need <= c->hist_cap && c->hist.p) return 0;
  const int cap = std::max(need + 4096, 2 * c->hist_cap);
  DBuf nb;
  int r = dalloc(c, nb, (size_t)cap * 4);
  if (r) return r;
  if (keep > 0) HIPCHK(hipMemcpyAsync(nb.p, c->hist.p, (size_t)keep * 4, hipMemcpyDeviceToDevice, c->st));
  HIPCHK(hipStreamSynchronize(c->st));
  std::swap(c->hist.p, nb.p);
  std::swap(c->hist.n, nb.n);
  c->hist_cap = cap;
  return 0;
}

int g4v_history_set(g4v_ctx* c, const int* toks, int L) {
  if (!c) return G4V_E_ARG;
  ARGCHK(L >= 0 && (L == 0 || toks), "history_set: L < 0 or null tokens");
  HIPCHK(hipSetDevice(c->device));
  int r = hist_reserve(c, L, 0);
  if (r) return r;
  if (L > 0) HIPCHK(hipMemcpyAsync(c->hist.p, toks, (size_t)L * 4, hipMemcpyHostToDevice, c->st));
  HIPCHK(hipStreamSynchronize(c->st));
  c->hist_len = L;
  return 0;
}

int g4v_prompt_lookup(g4v_ctx* c, const int* append, int na, int n, int maxlen, int* drafts, int* nd) {
  if (!c) return G4V_E_ARG;
  ARGCHK(na >= 0 && na <= PL_MAXA && (na == 0 || append), "prompt_lookup: 0 <= na <= 16 appended tokens");
  ARGCHK(n <= PL_MAXN, "prompt_lookup: n <= 256");
  ARGCHK(maxlen <= PL_MAXD, "prompt_lookup: maxlen <= 16");
  ARGCHK(nd && (maxlen <= 0 || drafts), "prompt_lookup: null output");
  ARGCHK(c->hist_len <= INT32_MAX - PL_MAXA, "prompt_lookup: history full");
  HIPCHK(hipSetDevice(c->device));
  int r = hist_reserve(c, c->hist_len + na, c->hist_len);
  if (r) return r;
  if (!c->plout.p) ALLOC(c->plout, (1 + PL_MAXD) * 4);
  if (!c->pl_host) HIPCHK(hipHostMalloc((void**)&c->pl_host, (1 + PL_MAXD) * 4, hipHostMallocDefault));
  PlAppend app{};
  app.n = na;
  for (int i = 0; i < na; ++i) app.t[i] = append[i];
  launch_prompt_lookup(c->hist.as<int>(), c->hist_len, app, n, std::max(maxlen, 0), c->plout.as<int>(), c->st);
  HIPCHK(hipGetLastError());
  HIPCHK(hipMemcpyAsync(c->pl_host, c->plout.p, (1 + PL_MAXD) * 4, hipMemcpyDeviceToHost, c->st));
  HIPCHK(hipStreamSynchronize(c->st));
  c->hist_len += na;
  *nd = c->pl_host[0];
  for (int i = 0; i < *nd; ++i) drafts[i] = c->pl_host[1 + i];
  return 0;
}

int g4v_history_read(g4v_ctx* c, int* toks, int cap, int* L) {
  if (!c || !L) return G4V_E_ARG;
  *L = c->hist_len;
  if (!toks || cap <= 0 || c->hist_len == 0) return 0;
  HIPCHK(hipSetDevice(c->device));
  HIPCHK(hipStreamSynchronize(c->st));
  HIPCHK(hipMemcpy(toks, c->hist.p, (size_t)std::min(cap, c->hist_len) * 4, hipMemcpyDeviceToHost));
  return 0;
}

int g4v_set_prefill_int8(g4v_ctx* c, int on) {
  if (!c) return G4V_E_ARG;
  c->pf_i8 = on != 0;
  return 0;
}

int g4v_set_decode_int8(g4v_ctx* c, int on) {
  if (!c) return G4V_E_ARG;
  c->dec_i8 = on != 0;
  return 0;
}

int g4v_set_draft_samepos(g4v_ctx* c, int on) {
  if (!c) return G4V_E_ARG;
  c->dr_same = on != 0;
  return 0;
}

int g4v_set_graphs(g4v_ctx* c, int on) {
  if (!c) return G4V_E_ARG;
  c->use_graph = on != 0;
  return 0;
}

// device read / copy bandwidth (the method of bench/stream_bw.cpp:10-19 on the GPU): a buffer of
// `bytes` streamed `passes` times after one warm-up pass, timed with events on the library stream
int g4v_hbm_stream(g4v_ctx* c, size_t bytes, int passes, int mode, double* gbps) {
  if (!c) return G4V_E_ARG;
  ARGCHK(gbps && bytes >= ((size_t)1 << 20) && bytes % 16 == 0 && passes >= 1 && passes <= 1000 &&
             (mode == 0 || mode == 1),
         "hbm_stream: bytes >= 1 MiB, a multiple of 16; 1 <= passes <= 1000; mode 0 (read) or 1 (copy)");
  HIPCHK(hipSetDevice(c->device));
  hipStream_t st = c->st;
  DBuf src, dst;
  ALLOC(src, bytes);
  ALLOC(dst, mode == 1 ? bytes : (size_t)stream_grid() * 256 * 16);
  const size_t n16 = bytes / 16;
  launch_stream(2, nullptr, src.as<uint4>(), n16, st);
  launch_stream(mode, src.as<uint4>(), dst.as<uint4>(), n16, st);
  HIPCHK(hipGetLastError());  // the fill and warm-up launches
  struct Events {  // destroyed on every return path
    hipEvent_t e[2] = {nullptr, nullptr};
    ~Events() {
      for (hipEvent_t x : e)
        if (x) (void)hipEventDestroy(x);
    }
  } ev;
  HIPCHK(hipEventCreate(&ev.e[0]));
  HIPCHK(hipEventCreate(&ev.e[1]));
  HIPCHK(hipEventRecord(ev.e[0], st));
  for (int p = 0; p < passes; ++p) launch_stream(mode, src.as<uint4>(), dst.as<uint4>(), n16, st);
  HIPCHK(hipGetLastError());
  HIPCHK(hipEventRecord(ev.e[1], st));
  HIPCHK(hipEventSynchronize(ev.e[1]));
  float ms = 0.f;
  HIPCHK(hipEventElapsedTime(&ms, ev.e[0], ev.e[1]));
  *gbps = (double)passes * (double)bytes * (mode == 1 ? 2.0 : 1.0) / ((double)ms * 1e-3) / 1e9;
  return 0;
}

// ---- the components on their own, device-timed: one launch (or launch pair) at a time between
// two events on the library's stream.  Warm: the launches repeat on the same operands, which stay
// in the caches (4 MB L2 per XCD, 256 MB last-level cache).  Cold: before each timed launch a
// read of a 512 MB buffer (twice the last-level cache) evicts them, outside the events.
static int time_launches(g4v_ctx* c, int iters, int cold, const std::function<void()>& launch, float* us) {
  hipStream_t st = c->st;
  DBuf src, dst;
  const size_t ebytes = (size_t)512 << 20, n16 = ebytes / 16;
  if (cold) {
    ALLOC(src, ebytes);
    ALLOC(dst, (size_t)stream_grid() * 256 * 16);
    launch_stream(2, nullptr, src.as<uint4>(), n16, st);
  }
  launch();  // warm-up (and code load)
  HIPCHK(hipGetLastError());
  struct Events {
    hipEvent_t e[2] = {nullptr, nullptr};
    ~Events() {
      for (hipEvent_t x : e)
        if (x) (void)hipEventDestroy(x);
    }
  } ev;
  HIPCHK(hipEventCreate(&ev.e[0]));
  HIPCHK(hipEventCreate(&ev.e[1]));
  double tot = 0;
  for (int i = 0; i < iters; ++i) {
    if (cold) launch_stream(0, src.as<uint4>(), dst.as<uint4>(), n16, st);
    HIPCHK(hipEventRecord(ev.e[0], st));
    launch();
    HIPCHK(hipEventRecord(ev.e[1], st));
    HIPCHK(hipEventSynchronize(ev.e[1]));
    float ms = 0.f;
    HIPCHK(hipEventElapsedTime(&ms, ev.e[0], ev.e[1]));
    tot += ms;
  }
  HIPCHK(hipGetLastError());
  *us = (float)(tot * 1000.0 / iters);
  return 0;
}

int g4v_w4g32_time(g4v_ctx* c, int nmat, const int* h, int M, int iters, int flags, float* us) {
  if (!c) return G4V_E_ARG;
  const int cold = flags & 1;
  const bool a8 = (flags & 2) != 0;
  ARGCHK(nmat >= 1 && nmat <= 3 && h && us && M >= 1 && M <= MAXM && iters >= 1 && iters <= 10000,
         "w4g32_time: 1 to 3 matrices, 1 <= M <= 8, 1 <= iters <= 10000");
  size_t ntot = 0;
  for (int j = 0; j < nmat; ++j) {
    ARGCHK(h[j] >= 0 && h[j] < (int)c->mats.size(), "w4g32_time: bad handle");
    ARGCHK(c->mats[h[j]]->K == c->mats[h[0]]->K && c->mats[h[j]]->N % 64 == 0,
           "w4g32_time: the matrices need the same K and N % 64 == 0");
    ntot += c->mats[h[j]]->N;
  }
  HIPCHK(hipSetDevice(c->device));
  const int K = c->mats[h[0]]->K;
  for (int j = 0; j < nmat; ++j) {  // the row-tiled copies, once per handle
    Mat& m = *c->mats[h[j]];
    ARGCHK(!a8 || m.a8w.p, "w4g32_time: W4A8 needs the matrices' operand tiles (N % 16 == 0)");
    if (!a8 && !m.tw.p) {
      ALLOC(m.tw, (size_t)m.N * m.K / 2);
      ALLOC(m.ts, (size_t)m.N * m.K / 16);
      launch_tile_w4(m.wr.as<uint4>(), m.s.as<uint16_t>(), m.tw.as<uint4>(), m.ts.as<uint4>(), m.N, m.K, c->st);
    }
  }
  if (c->gx.n < (size_t)MAXM * K * 4) ALLOC(c->gx, (size_t)MAXM * K * 4);
  if (c->gy.n < (size_t)M * ntot * 4) ALLOC(c->gy, (size_t)MAXM * ntot * 4);
  HIPCHK(hipMemsetAsync(c->gx.p, 0, (size_t)M * K * 4, c->st));  // staged rows (values do not matter)
  GemvTArgs a{};
  size_t off = 0;
  for (int j = 0; j < nmat; ++j) {
    const Mat& m = *c->mats[h[j]];
    a.mat[j] = a8 ? W4Tile{m.a8w.as<uint4>(), m.a8s.as<uint4>(), m.N} : m.tile();
    a.y[j] = c->gy.as<float>() + off;
    a.ldy[j] = m.N;
    off += (size_t)M * m.N;
  }
  a.xs = c->gx.as<float4>();
  a.K = K;
  a.M = M;
  // the verify pass's launch shapes: one row a block at M = 1 (32-row tiles; plain products of
  // K % 2048 == 0 on the one-row kernel), else 2 rows (4 for a pair, 1 past K 1536) on 64-row tiles;
  // W4A8: the verify pass's product of staged rows (quantised in its blocks)
  const int mpl = M == 1 ? 1 : (nmat >= 2 ? std::min(4, M) : (K > H ? 1 : 2)), tr = M == 1 ? 32 : 64;
  if (a8) ARGCHK(K % 256 == 0, "w4g32_time: W4A8 needs K % 256 == 0");
  return time_launches(c, iters, cold, [&] {
    if (a8)
      (void)launch_gemv_a8(a, c->st);
    else
      (void)launch_gemv_t(a, c->st, mpl, tr);
  }, us);
}

int g4v_attn_time(g4v_ctx* c, int npos, int M, int nsplit, int window, int iters, int cold, float* us) {
  if (!c) return G4V_E_ARG;
  ARGCHK(us && npos >= M && npos <= 65536 && M >= 1 && M <= MAXM && nsplit >= 1 && nsplit <= MAXT && iters >= 1 &&
             iters <= 10000,
         "attn_time: M <= npos <= 65536, 1 <= M <= 8, 1 <= nsplit <= 16, 1 <= iters <= 10000");
  AttnGeom g{};
  g.M = M;
  g.kmax = npos - 1;
  g.kmin = g.kmax;
  g.T = nsplit;
  for (int m = 0; m < M; ++m) {
    g.pos[m] = npos - M + m;
    g.lo[m] = window ? std::max(0, g.pos[m] - 511) : 0;
    g.skip_lo[m] = 1;
    g.skip_hi[m] = 0;
    g.kmin = std::min(g.kmin, g.lo[m]);
  }
  const int len = g.kmax - g.kmin + 1;
  ARGCHK((len + nsplit - 1) / nsplit <= attn_pmax(), "attn_time: more positions per split than the split buffer holds");
  HIPCHK(hipSetDevice(c->device));
  const size_t kvb = (size_t)kv_cap(npos) * HD * 2;
  if (c->ak.n < kvb) ALLOC(c->ak, kvb);
  if (c->av.n < kvb) ALLOC(c->av, kvb);
  if (c->aq.n < (size_t)MAXM * NQ * HD * 4) ALLOC(c->aq, (size_t)MAXM * NQ * HD * 4);
  if (c->ao.n < (size_t)MAXM * NQ * HD * 4) ALLOC(c->ao, (size_t)MAXM * NQ * HD * 4);
  if (c->po.n < (size_t)MAXT * MAXM * NQ * HD * 4) {
    drop_graphs(c);  // the split partials are shared with the captured verify steps
    ALLOC(c->po, (size_t)MAXT * MAXM * NQ * HD * 4);
    ALLOC(c->pm, (size_t)MAXT * MAXM * NQ * 4);
    ALLOC(c->pl, (size_t)MAXT * MAXM * NQ * 4);
  }
  // finite operands (bf16 0x3c3c, fp32 0x3c3c3c3c): the values do not change the work
  HIPCHK(hipMemsetAsync(c->ak.p, 0x3c, kvb, c->st));
  HIPCHK(hipMemsetAsync(c->av.p, 0x3c, kvb, c->st));
  HIPCHK(hipMemsetAsync(c->aq.p, 0x3c, (size_t)M * NQ * HD * 4, c->st));
  return time_launches(c, iters, cold, [&] {
    launch_attn_geom(c->ak.as<uint16_t>(), c->av.as<uint16_t>(), c->aq.as<float>(), NQ * HD, g, c->po.as<float>(),
                     c->pm.as<float>(), c->pl.as<float>(), c->ao.as<float>(), NQ * HD, c->st);
  }, us);
}

int g4v_head_time(g4v_ctx* c, const float* h, int iters, int cold, float* us, int* nsurv, int* fallback) {
  if (!c) return G4V_E_ARG;
  if (!c->head_ready) {
    c->err = "head_time: no head (g4v_head_build or g4v_model_synth first)";
    return G4V_E_STATE;
  }
  ARGCHK(h && us && iters >= 1 && iters <= 10000, "head_time: need h and 1 <= iters <= 10000");
  int G = 0, ns = 0, fb = 0;
  int r = g4v_head_argmax(c, h, 1, &G, &ns, &fb);  // uploads the row and its norm (E:1417)
  if (r) return r;
  if (nsurv) *nsurv = ns;
  if (fallback) *fallback = fb;
  return time_launches(c, iters, cold, [&] {
    head_run(head_args(c, c->hb1, c->hrow.as<float>(), c->hnrow.as<float>(), 1, nullptr), c->st);
  }, us);
}

int g4v_sync(g4v_ctx* c) {
  if (!c) return G4V_E_ARG;
  HIPCHK(hipSetDevice(c->device));
  HIPCHK(hipStreamSynchronize(c->st));
  HIPCHK(hipDeviceSynchronize());
  return 0;
}

int g4v_profile(g4v_ctx* c, unsigned mask) {
  if (!c) return G4V_E_ARG;
  c->prof_mask = mask;
  c->recs.clear();
  c->evused = 0;
  for (int t = 0; t < PT_NTAGS; ++t) {
    c->prof_ms[t] = 0;
    c->prof_bytes[t] = 0;
    c->prof_n[t] = 0;
  }
  return 0;
}

int g4v_prefill_head_stats(g4v_ctx* c, int* nsurv, int* fallback) {
  if (!c) return G4V_E_ARG;
  if (nsurv) *nsurv = c->pf_nsurv;
  if (fallback) *fallback = c->pf_fallback;
  return 0;
}

int g4v_profile_read(g4v_ctx* c, double* ms, double* bytes, long long* count, int n) {
  if (!c || n < 0) return G4V_E_ARG;
  for (int t = 0; t < n && t < PT_NTAGS; ++t) {
    if (ms) ms[t] = c->prof_ms[t];
    if (bytes) bytes[t] = c->prof_bytes[t];
    if (count) count[t] = c->prof_n[t];
  }
  return PT_NTAGS;
}

long long g4v_expf_selftest(uint32_t lo, uint32_t hi, uint32_t stride) {
  static const uint64_t tab[32] = G4V_EXPF_TABLE;
  long long bad = 0;
  if (stride == 0) stride = 1;
  for (uint64_t u = lo; u <= hi; u += stride) {
    const float x = as_f32((uint32_t)u);
    if (!(x <= 0.0f)) continue;
    if (as_u32(libm_expf_neg(x, tab)) != as_u32(expf(x))) ++bad;
  }
  return bad;
}

}  // extern "C"
