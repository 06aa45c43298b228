// ref_harness.cpp -- C entry points into the reference engine's own kernels.
//
// TEST INFRASTRUCTURE.  Built by oracle/Makefile from the reference sources where
// they lie (the engine is included with `#define main engine_main`, the trick the
// reference's bench/attn_bench.cpp:2-4 uses); the output goes to oracle/_ref/ only.
// Used to pin the C oracle bit-for-bit and as the "reference" CPU baseline.
// Every wrapper calls the reference's static functions unchanged; the few lines
// that compose them restate the call sites they cite (E = engine/gemma4_engine.cpp).
#include <map>
#include <memory>
#define main engine_main
#include G4_REF_ENGINE
#undef main
#include <sched.h>

namespace {
XP g_xa, g_xb;
bool g_started = false;
// joins the pool's workers before the pool itself is destroyed at process exit
struct PoolStopper {
  ~PoolStopper() {
    if (g_started) POOL.shutdown();
  }
} g_stopper;
}

extern "C" {

// Start the reference's worker pool with T threads on CPUs 0..T-1 (E:75-77), then give the
// calling thread its original affinity back (the pool pins its caller to cpus[0]).
int ref_start(int T) {
  if (g_started) return POOL.T;
  cpu_set_t keep;
  CPU_ZERO(&keep);
  pthread_getaffinity_np(pthread_self(), sizeof keep, &keep);
  std::vector<int> cpus;
  for (int c = 0; c < CPU_SETSIZE && (int)cpus.size() < T; ++c)
    if (CPU_ISSET(c, &keep)) cpus.push_back(c);
  if (cpus.empty()) cpus.push_back(0);
  POOL.start(cpus);
  pthread_setaffinity_np(pthread_self(), sizeof keep, &keep);
  g_started = true;
  return POOL.T;
}

// the pool on the given CPUs (the engine's ENGINE_CPUS list, E:1216-1217)
int ref_start_cpus(const int* cpus, int n) {
  if (g_started) return POOL.T;
  cpu_set_t keep;
  CPU_ZERO(&keep);
  pthread_getaffinity_np(pthread_self(), sizeof keep, &keep);
  std::vector<int> v(cpus, cpus + std::max(1, std::min(n, 16)));
  POOL.start(v);
  pthread_setaffinity_np(pthread_self(), sizeof keep, &keep);
  g_started = true;
  return POOL.T;
}

int ref_threads(void) { return POOL.active_count(); }

// W4G32 through the engine's XP::prep + lin1 (E:180-194, 241-255, 310-317), exact-float mode
void ref_w4g32(const uint8_t* W, const uint16_t* S, const float* X, int M, int N, int K, float* Y) {
  G_I8_ACTIVE = false;
  g_xa.prep(X, K, M);
  Q4 q;
  q.w = W;
  q.s = S;
  q.N = N;
  q.K = K;
  lin1(g_xa, q, Y);
}

// W4A8: repack (A8:18-27), quant (A8:30-42) and tiles of 4 + remainder as i8_task does (E:304-309)
void ref_w4a8(const uint8_t* W, const uint16_t* S, const float* X, int M, int N, int K, float* Y,
              int8_t* q, float* sx, int32_t* sum) {
  w4a8::Packed P;
  w4a8::repack_alloc(N, K, P);
  w4a8::repack_tiles(W, S, N, K, P, 0, N / 8);
  w4a8::XQ xq;
  w4a8::quant(X, M, K, xq);
  for (int t = 0; t < N / 8; ++t) {
    int m = 0;
    for (; m + 4 <= M; m += 4) w4a8::tile<4>(P, t, xq, m, Y);
    for (; m < M; ++m) w4a8::tile<1>(P, t, xq, m, Y);
  }
  const int G = K / 32;
  if (q) std::memcpy(q, xq.q.data(), (size_t)M * K);
  if (sx) std::memcpy(sx, xq.sx.data(), sizeof(float) * (size_t)M * G);
  if (sum) std::memcpy(sum, xq.sum.data(), sizeof(int32_t) * (size_t)M * G);
}

void ref_exp8(const float* x, int n, float* y) {
  for (int i = 0; i + 8 <= n; i += 8) _mm256_storeu_ps(y + i, exp8(_mm256_loadu_ps(x + i)));  // n % 8 == 0
}
void ref_gelu8(const float* x, int n, float* y) {
  for (int i = 0; i + 8 <= n; i += 8) _mm256_storeu_ps(y + i, gelu8(_mm256_loadu_ps(x + i)));  // n % 8 == 0
}
void ref_rbf8(const float* x, int n, float* y) {
  for (int i = 0; i + 8 <= n; i += 8) _mm256_storeu_ps(y + i, rbf8(_mm256_loadu_ps(x + i)));  // n % 8 == 0
}
void ref_f2bf(const float* x, int n, uint16_t* y) {
  for (int i = 0; i < n; ++i) y[i] = f2bf(x[i]);
}
double ref_ss(const float* x, int n) { return ss_avx2(x, n); }
void ref_rms(const float* x, const float* w, int n, float* y) { rms(x, w, n, y); }
void ref_rms_r16_inplace(float* x, const float* w, int n) { rms_r16_inplace(x, w, n); }
void ref_rms_prep_x(const float* x, const float* w, int n, float* y, float* xe, float* xo, float* gs,
                    int r16) {
  rms_prep_x(x, w, n, y, xe, xo, gs, r16 != 0);
}
void ref_add_res_prep_x(float* x, const float* y, int n, float* xe, float* xo, float* gs) {
  add_res_prep_x(x, y, n, xe, xo, gs);
}
void ref_add_res_inplace(float* x, const float* y, int n) { add_res_inplace(x, y, n); }
void ref_rope(float* h, const float* cs, const float* sn, int hd) { rope_avx2(h, cs, sn, hd); }
void ref_prep_x(const float* x, int K, float* xe, float* xo, float* gs) { prep_x_avx2(x, K, xe, xo, gs); }
float ref_calc_thr(float L) { return calc_thr_fast(L); }

// gate/up GEMV + gelu + prep of the down input (E:256-302), one worker (tid 0 of 1)
void ref_gate_up(const uint8_t* Wg, const uint16_t* Sg, const uint8_t* Wu, const uint16_t* Su, int I,
                 int K, const float* X, int M, float* gbuf, float* ubuf, float* xe, float* xo,
                 float* gs) {
  g_xa.prep(X, K, M);
  Q4 g, u;
  g.w = Wg; g.s = Sg; g.N = I; g.K = K;
  u.w = Wu; u.s = Su; u.N = I; u.K = K;
  std::vector<float> abuf((size_t)M * I);
  g_xb.K = I;
  g_xb.M = M;
  GateUpArg a{&g_xa, &g, &u, gbuf, ubuf, abuf.data(), &g_xb};
  gate_up_fused_task(&a, 0, 1);
  for (int m = 0; m < M; ++m) {
    std::memcpy(xe + (size_t)m * I / 2, g_xb.xe + (size_t)m * I / 2, sizeof(float) * I / 2);
    std::memcpy(xo + (size_t)m * I / 2, g_xb.xo + (size_t)m * I / 2, sizeof(float) * I / 2);
    std::memcpy(gs + (size_t)m * I / 32, g_xb.gs + (size_t)m * I / 32, sizeof(float) * I / 32);
  }
}

// split-KV attention: every split t of T in turn (E:743-877), then attn_merge (E:1019-1059);
// out receives the rounded outputs, xe/xo/gs (optional) the fused o_proj prep.  M <= 4.
// Returns -1 (nothing computed) outside the reference's capacity: AttnArg holds 4 rows
// (E:739), the partial buffers 16 splits of hd <= 512, a split at most ACH = 8192 positions.
int ref_attn(const uint16_t* Kc, const uint16_t* Vc, int hd, int nh, int M, const float* q, int ldq,
             const int* pos, const int* lo, const int* skip_lo, const int* skip_hi, int kmin,
             int kmax, int T, float* out, int ldo, float* xe, float* xo, float* gs, float* part_m,
             float* part_l) {
  if (M < 1 || M > 4 || T < 1 || T > 16 || hd > 512 || nh > 8 || kmax < kmin ||
      (kmax - kmin + 1 + T - 1) / T > ACH)
    return -1;
  G_I8_ACTIVE = false;
  AttnArg aa;
  aa.Kc = Kc;
  aa.Vc = Vc;
  aa.hd = hd;
  aa.nh = nh;
  aa.M = M;
  aa.kmin = kmin;
  aa.kmax = kmax;
  float* outp[4];
  for (int m = 0; m < M; ++m) {
    aa.q[m] = q + (size_t)m * ldq;
    aa.pos[m] = pos[m];
    aa.lo[m] = lo[m];
    aa.skip_lo[m] = skip_lo[m];
    aa.skip_hi[m] = skip_hi[m];
    outp[m] = out + (size_t)m * ldo;
  }
  for (int t = 0; t < T; ++t) attn_task(&aa, t, T);
  if (part_m)
    for (int t = 0; t < T; ++t)
      for (int m = 0; m < M; ++m)
        for (int h = 0; h < nh; ++h) {
          part_m[((size_t)t * M + m) * nh + h] = A_M[t][m][h];
          part_l[((size_t)t * M + m) * nh + h] = A_L[t][m][h];
        }
  attn_merge(aa, T, outp, nullptr);
  if (xe) {
    attn_merge(aa, T, outp, &g_xb);
    const int K = nh * hd;
    for (int m = 0; m < M; ++m) {
      std::memcpy(xe + (size_t)m * K / 2, g_xb.xe + (size_t)m * K / 2, sizeof(float) * K / 2);
      std::memcpy(xo + (size_t)m * K / 2, g_xb.xo + (size_t)m * K / 2, sizeof(float) * K / 2);
      std::memcpy(gs + (size_t)m * K / 32, g_xb.gs + (size_t)m * K / 32, sizeof(float) * K / 32);
    }
  }
  return 0;
}

// The screen scan (E:460-538) over the 262,144 x 1536 screen with one worker.  h: M <= 4 rows
// (bf16-valued), seedL: the pre-screen lower bound per row (E:1445-1449).  Outputs per row:
// candidate count / indices / U values (capacity 16384 each), the max lower bound, overflow.
int ref_screen(const uint8_t* Wq, const uint16_t* Sq, const float* coef, const float* h, int M,
               const float* seedL, int* cnt, int* idx, float* u, float* tmax, int* overflow) {
  static Screen S;
  S.w.assign(Wq, Wq + (size_t)262144 * 768);
  S.s.assign(Sq, Sq + (size_t)262144 * 48);
  S.coef.assign(coef, coef + 262144);
  S.on = true;
  static float hn[4];
  g_xa.prep(h, 1536, M);
  for (int m = 0; m < M; ++m) hn[m] = (float)sqrt(ss_avx2(h + (size_t)m * 1536, 1536));
  ScrArg* SA = new ScrArg();
  for (int m = 0; m < M; ++m) {
    SA->pre_thr[m] = seedL[m];
    SA->shared_best[m].store(seedL[m], std::memory_order_relaxed);
    SA->overflow[m].store(false, std::memory_order_relaxed);
  }
  SA->S = &S;
  SA->x = &g_xa;
  SA->hn = hn;
  SA->M = M;
  SA->nxt.store(0, std::memory_order_relaxed);
  screen_task(SA, 0, 1);
  for (int m = 0; m < M; ++m) {
    cnt[m] = SA->t_cnt[0][m];
    std::memcpy(idx + (size_t)m * 16384, SA->t_idx[0][m], sizeof(int) * 16384);
    std::memcpy(u + (size_t)m * 16384, SA->t_u[0][m], sizeof(float) * 16384);
    tmax[m] = SA->tmax[0][m];
    overflow[m] = SA->overflow[m].load() ? 1 : 0;
  }
  delete SA;
  return 0;
}

// exp3 pack (X3:26-49); counts first (data == nullptr returns the exception count)
namespace {
bf16p::Packed g_hp;
}
int64_t ref_exp3_pack(const uint16_t* W, int N, int K, const uint8_t* cb8) {
  bf16p::pack(W, N, K, cb8, g_hp);
  return (int64_t)g_hp.exc_col.size();
}
void ref_exp3_get(uint8_t* data, int64_t* exc_ptr, uint16_t* exc_col, float* exc_delta) {
  std::memcpy(data, g_hp.data.data(), g_hp.data.size());
  std::memcpy(exc_ptr, g_hp.exc_ptr.data(), sizeof(int64_t) * g_hp.exc_ptr.size());
  std::memcpy(exc_col, g_hp.exc_col.data(), sizeof(uint16_t) * g_hp.exc_col.size());
  std::memcpy(exc_delta, g_hp.exc_delta.data(), sizeof(float) * g_hp.exc_delta.size());
}

// exact rescore of a survivor list (E:539-571) with one worker, on the last packed head
float ref_resc(const float* h, const int* idx, int cnt, float* fval) {
  RescArg RA;
  RA.P = &g_hp;
  RA.h = h;
  RA.fval = fval;
  RA.idx = idx;
  RA.cnt = cnt;
  resc_task(&RA, 0, 1);
  return RA.tmax[0];
}

// full head (E:573-579) over the last packed head, M <= 4 rows, logit [M][N]
void ref_head(const float* h, int M, float* logit) {
  HeadArg HA;
  HA.P = &g_hp;
  HA.h = h;
  HA.logit = logit;
  HA.M = M;
  head_task(&HA, 0, 1);
}

// ---------------------------------------------------------------------------------------
// One verify pass of the synthetic stack run by the reference's own kernels on its pool:
// the call sequence restates fwd (E:1262-1405, per-layer-embedding branch zero, every layer
// owning its KV), head_group (E:1408-1500) and the acceptance step (E:1647-1661), extended
// to two draft branches exactly as the C oracle does.  Used as the "reference" CPU baseline
// and to pin the oracle's layer composition.
// ---------------------------------------------------------------------------------------
struct RefLayer {
  const uint8_t* W[7];
  const uint16_t* S[7];
  const float* nv[6];  // in_ln, post_attn, pre_ff, post_ff, qn, kn
  float scalar;
  int sliding;
};
struct RefModel {
  int V, NL, I, ctx;
  const uint16_t* E;
  const float* fnorm;
  uint16_t* KC;  // [NL][ctx][256]
  uint16_t* VC;
  const float* cs[2];
  const float* sn[2];
  RefLayer L[64];
};
struct RefOut {
  int nacc, branch, ncommit;
  int commit[8], G[8], fallback[8], nsurv[8];
};

namespace {
Screen g_scr;
XP g_xh;
}

// screen + exp3 head of a 262,144-row vocabulary (the screen scan hardcodes that size)
void ref_head_setup(const uint8_t* Wq, const uint16_t* Sq, const float* coef, const uint8_t* x3, const uint8_t* cb,
                    const int64_t* xptr, const uint16_t* xcol, const float* xdel, int V) {
  g_scr.w.assign(Wq, Wq + (size_t)V * 768);
  g_scr.s.assign(Sq, Sq + (size_t)V * 48);
  g_scr.coef.assign(coef, coef + V);
  g_scr.on = true;
  g_hp.N = V;
  g_hp.K = 1536;
  std::memset(g_hp.cb, 0, 16);
  std::memcpy(g_hp.cb, cb, 8);
  g_hp.data.assign(x3, x3 + (size_t)V * 48 * 44);
  g_hp.exc_ptr.assign(xptr, xptr + V + 1);
  g_hp.exc_col.assign(xcol, xcol + xptr[V]);
  g_hp.exc_delta.assign(xdel, xdel + xptr[V]);
}

// E:1408-1500 head_group over rows [hf, Mend) of hbuf; G receives the greedy tokens
static void head_group_ref(float (*hbuf)[1536], const int* toks, int M, int hf, int Mend, int chain_lazy, int* G,
                           int* fb, int* ns, int sibling = -1) {
  const int H = 1536, Mh = Mend - hf;
  auto cap = [](float s) { return r16(30.0f * tanhf(s / 30.0f)); };
  static ScrArg* SA = new ScrArg();
  static float hn[4];
  constexpr int LIM = 30000;
  static int fi[LIM];
  static float fval[LIM];
  static float logit[4][262144];
  g_xh.prep(&hbuf[hf][0], H, Mh);
  for (int m = 0; m < Mh; ++m) hn[m] = (float)sqrt(ss_avx2(hbuf[hf + m], H));
  float seed_L[4] = {-1e30f, -1e30f, -1e30f, -1e30f};
  int seeds[160], nseeds = 0;  // E:1419-1427 (no drafter: the fixed list)
  for (int m = 0; m < std::min(M, 8); ++m)
    if (toks[m] >= 0 && toks[m] < 262144) seeds[nseeds++] = toks[m];
  const int fixed_seeds[] = {2, 106, 107, 108, 235248, 235265, 235269, 476, 573, 577, 604, 651, 688, 728, 785, 818, 947, 1024, 1154, 1280};
  for (int s : fixed_seeds) seeds[nseeds++] = s;
  for (int si = 0; si < nseeds; ++si) {
    const int n = seeds[si];
    float sd[4];
    const uint8_t* Wn = g_scr.w.data() + (size_t)n * (H / 2);
    const uint16_t* Scn = g_scr.s.data() + (size_t)n * (H / 32);
    switch (Mh) {
      case 1: w4::gemm_rows_tile<1>(Wn, Scn, g_xh.xe, g_xh.xo, g_xh.gs, H, 0, 1, sd, 1, H / 2, H / 32); break;
      case 2: w4::gemm_rows_tile<2>(Wn, Scn, g_xh.xe, g_xh.xo, g_xh.gs, H, 0, 1, sd, 1, H / 2, H / 32); break;
      case 3: w4::gemm_rows_tile<3>(Wn, Scn, g_xh.xe, g_xh.xo, g_xh.gs, H, 0, 1, sd, 1, H / 2, H / 32); break;
      default: w4::gemm_rows_tile<4>(Wn, Scn, g_xh.xe, g_xh.xo, g_xh.gs, H, 0, 1, sd, 1, H / 2, H / 32); break;
    }
    const float c = g_scr.coef[n];
    for (int m = 0; m < Mh; ++m) seed_L[m] = std::max(seed_L[m], sd[m] - c * hn[m]);
  }
  for (int m = 0; m < Mh; ++m) {
    SA->pre_thr[m] = seed_L[m];
    SA->shared_best[m].store(seed_L[m], std::memory_order_relaxed);
    SA->overflow[m].store(false, std::memory_order_relaxed);
  }
  SA->S = &g_scr;
  SA->x = &g_xh;
  SA->hn = hn;
  SA->M = Mh;
  SA->nxt.store(0, std::memory_order_relaxed);
  POOL.run(screen_task, SA);
  const int actT = POOL.active_count();
  float Lm[4];
  for (int m = 0; m < Mh; ++m) {
    float L = -1e30f;
    for (int t = 0; t < actT; ++t) L = std::max(L, SA->tmax[t][m]);
    Lm[m] = L;
  }
  static RescArg RA;
  auto eval_row = [&](int m) -> bool {  // E:1453-1474
    if (SA->overflow[m].load(std::memory_order_relaxed)) return false;
    const float thr = calc_thr_fast(Lm[m]);
    int tot = 0;
    for (int t = 0; t < actT; ++t)
      for (int k = 0; k < SA->t_cnt[t][m]; ++k)
        if (SA->t_u[t][m][k] >= thr) {
          if (tot >= LIM) return false;
          fi[tot++] = SA->t_idx[t][m][k];
        }
    RA.P = &g_hp;
    RA.h = hbuf[hf + m];
    RA.fval = fval;
    RA.idx = fi;
    RA.cnt = tot;
    POOL.run(resc_task, &RA);
    float mx = -1e30f;
    for (int t = 0; t < actT; ++t) mx = std::max(mx, RA.tmax[t]);
    const float cm = cap(mx);
    int best = -1;
    for (int i = 0; i < tot; ++i)
      if (fval[i] >= mx - 2.0f && cap(fval[i]) == cm) {
        best = fi[i];
        break;
      }
    G[hf + m] = best;
    ns[hf + m] = tot;
    return true;
  };
  bool ok = true;
  if (chain_lazy && Mh > 1) {  // E:1475-1484: the chain rows, or the sibling row when it holds G[0]
    if (!eval_row(0)) ok = false;
    else if (sibling > 0 && G[0] != toks[1] && G[0] == toks[sibling]) {
      if (!eval_row(sibling)) ok = false;
    } else {
      const int chain_end = sibling > 0 ? sibling : Mh;
      for (int m = 1; m < chain_end; ++m) {
        if (G[hf + m - 1] != toks[hf + m]) break;
        if (!eval_row(m)) {
          ok = false;
          break;
        }
      }
    }
  } else {
    for (int m = 0; m < Mh; ++m)
      if (!eval_row(m)) {
        ok = false;
        break;
      }
  }
  if (!ok) {  // E:1489-1498 full head for the whole group
    HeadArg HA;
    HA.P = &g_hp;
    HA.h = &hbuf[hf][0];
    HA.logit = &logit[0][0];
    HA.M = Mh;
    POOL.run(head_task, &HA);
    for (int m = 0; m < Mh; ++m) {
      float* lg = &logit[0][0] + (size_t)m * 262144;
      float mx = -1e30f;
      for (int i = 0; i < 262144; ++i) {
        lg[i] = r16(lg[i]);
        mx = std::max(mx, lg[i]);
      }
      const float cm = cap(mx);
      int best = -1;
      for (int i = 0; i < 262144; ++i)
        if (lg[i] >= mx - 2.0f && cap(lg[i]) == cm) {
          best = i;
          break;
        }
      G[hf + m] = best;
      fb[hf + m] = 1;
    }
  }
}


// ---------------------------------------------------------------------------------------
// Prefill attention and the prefill pass (E:1594-1599 with ENGINE_PREFILL_INT8=1)
// ---------------------------------------------------------------------------------------
// attn_tile (E:1063-1083) over rows at pos0 .. pos0+M-1, tiles of QB in turn on worker slot 0
void ref_attn_tile(const uint16_t* Kc, const uint16_t* Vc, int sliding, const float* q, int pos0, int M, float* att) {
  for (int t = 0; t < (M + QB - 1) / QB; ++t) attn_tile(Kc, Vc, 256, sliding != 0, q, 2048, pos0, M, att, t, 0);
}

// run_mh (E:1338-1349) on already normed and rotated q, as the lambda does it; sibling >= 0: that
// row's window starts from position pos0 + 1 and it skips the rows between row 0 and itself (E:1345)
static void run_mh_rows(const uint16_t* Kc, const uint16_t* Vc, int sliding, const float* q, int pos0, int M,
                        float* att, int sibling = -1) {
  const int hd = 256;
  std::vector<float> scv((size_t)pos0 + M + 8);
  float* sc = scv.data();
  for (int mh = 0; mh < M * 8; ++mh) {
    const int m = mh / 8, h = mh % 8, cachepos = pos0 + m, pos = m == sibling ? pos0 + 1 : cachepos;
    const float* qh = q + (size_t)m * 2048 + h * hd;
    const int lo = sliding ? std::max(0, pos - 511) : 0;
    auto valid = [&](int p) { return m != sibling || p <= pos0 || p == cachepos; };
    float mx = -1e30f;
    for (int p = lo; p <= cachepos; ++p) {
      if (!valid(p)) continue;
      __m256 sv = _mm256_setzero_ps();
      const uint16_t* kp = Kc + (size_t)p * hd;
      for (int i = 0; i < hd; i += 8) sv = _mm256_fmadd_ps(_mm256_loadu_ps(qh + i), bf8(kp + i), sv);
      float d = w4::hsum(sv);
      sc[p] = d;
      mx = std::max(mx, d);
    }
    float den = 0;
    for (int p = lo; p <= cachepos; ++p) {
      if (!valid(p)) continue;
      sc[p] = expf(sc[p] - mx);
      den += sc[p];
    }
    float* oh = att + (size_t)m * 8 * hd + h * hd;
    for (int i = 0; i < hd; ++i) oh[i] = 0;
    for (int p = lo; p <= cachepos; ++p) {
      if (!valid(p)) continue;
      float wgt = sc[p] / den;
      const uint16_t* vp = Vc + (size_t)p * hd;
      for (int i = 0; i < hd; i += 8)
        _mm256_storeu_ps(oh + i, _mm256_fmadd_ps(_mm256_set1_ps(wgt), bf8(vp + i), _mm256_loadu_ps(oh + i)));
    }
    rbf_n(oh, hd);
  }
}
void ref_attn_mh(const uint16_t* Kc, const uint16_t* Vc, int sliding, const float* q, int pos0, int M, float* att) {
  run_mh_rows(Kc, Vc, sliding, q, pos0, M, att);
}

namespace {
std::map<const uint8_t*, std::unique_ptr<w4a8::Packed>> g_pk;  // W4A8 repack of each matrix, once
const w4a8::Packed* packed(const uint8_t* W, const uint16_t* S, int N, int K) {
  auto& p = g_pk[W];
  if (!p) {
    p.reset(new w4a8::Packed());
    w4a8::repack_alloc(N, K, *p);
    w4a8::repack_tiles(W, S, N, K, *p, 0, N / 8);
  }
  return p.get();
}
}  // namespace

void ref_pack_reset(void) { g_pk.clear(); }

// The prefill loop of run_req (E:1594-1599) over the synthetic stack with G_I8_ACTIVE = G_I8 =
// true: fwd (E:1256-1405) per block of at most pfb rows, the engine's attention-path choice
// (E:1305, 1328, 1337 with SPLITKV, TILED, ATT_PAR = 192) and lin_multi's W4A8 rule (M >= 2,
// E:311).  hlast receives the last row's r16(rms(x, fnorm)).  Returns -1 for pfb outside 1..32.
int ref_prefill_ex(RefModel* md, const int* toks, int n, int pos0, int pfb, int i8, float* hlast);
int ref_prefill(RefModel* md, const int* toks, int n, int pos0, int pfb, float* hlast) {
  return ref_prefill_ex(md, toks, n, pos0, pfb, 1, hlast);
}
// i8: G_I8 (ENGINE_PREFILL_INT8=1, E:1210), the prompt's blocks of two rows or more multiply
// W4A8; 0: exact float throughout (G_I8_ACTIVE false, E:1363)
int ref_prefill_ex(RefModel* md, const int* toks, int n, int pos0, int pfb, int i8, float* hlast) {
  if (pfb < 1 || pfb > 32) return -1;
  const int H = 1536, NL = md->NL, I = md->I;
  const int T = POOL.active_count();
  alignas(64) static float x[32][1536], a[32][1536], mlp_in[32][1536], q[32][2048], k[32][256], v[32][256],
      att[32][2048], o[32][1536], tmp[1536];
  static std::vector<float> gbuf, ubuf, abuf;
  gbuf.resize((size_t)32 * I);
  ubuf.resize((size_t)32 * I);
  abuf.resize((size_t)32 * I);
  static XP XA, XB;
  const __m256 vsqh = _mm256_set1_ps(sqrtf((float)H));
  G_I8_ACTIVE = i8 != 0;
  for (int done = 0; done < n;) {
    const int M = std::min(pfb, n - done), p0 = pos0 + done;
    const bool last = done + M == n;
    const int* tk = toks + done;
    const bool split = M <= 4 && p0 + M > 192, tiled = !split && M >= 4 && p0 + M > 64;
    for (int m = 0; m < M; ++m) {  // E:1262-1267
      const uint16_t* er = md->E + (size_t)tk[m] * H;
      for (int i = 0; i < H; i += 8) _mm256_storeu_ps(x[m] + i, rbf8(_mm256_mul_ps(bf8(er + i), vsqh)));
      rms_prep_x(x[m], md->L[0].nv[0], H, a[m], XA.xe + (size_t)m * (H / 2), XA.xo + (size_t)m * (H / 2),
                 XA.gs + (size_t)m * (H / 32), false);
    }
    XA.K = H;
    XA.M = M;
    XA.src = &a[0][0];
    XA.qdone = false;
    for (int l = 0; l < NL; ++l) {
      const RefLayer& A = md->L[l];
      Q4 qm[7];
      const int Ns[7] = {2048, 256, 256, 1536, I, I, 1536}, Ks[7] = {1536, 1536, 1536, 2048, 1536, 1536, I};
      for (int j = 0; j < 7; ++j) {
        qm[j].w = A.W[j];
        qm[j].s = A.S[j];
        qm[j].N = Ns[j];
        qm[j].K = Ks[j];
        qm[j].p8 = packed(A.W[j], A.S[j], Ns[j], Ks[j]);
      }
      {  // E:1289
        const Q4* qq[3] = {&qm[0], &qm[1], &qm[2]};
        float* yy[3] = {&q[0][0], &k[0][0], &v[0][0]};
        lin_multi(XA, 3, qq, yy);
      }
      const int ty = A.sliding ? 0 : 1;
      uint16_t* KCl = md->KC + (size_t)l * md->ctx * 256;
      uint16_t* VCl = md->VC + (size_t)l * md->ctx * 256;
      for (int m = 0; m < M; ++m) {  // E:1291-1303 / 1307-1324 / 1331-1334 / 1343-1344
        const float* cs = md->cs[ty] + (size_t)(p0 + m) * 128;
        const float* sn = md->sn[ty] + (size_t)(p0 + m) * 128;
        for (int h = 0; h < 8; ++h) {
          rms_r16_inplace(q[m] + h * 256, A.nv[4], 256);
          rope_avx2(q[m] + h * 256, cs, sn, 256);
        }
        rms_r16_inplace(k[m], A.nv[5], 256);
        rope_avx2(k[m], cs, sn, 256);
        rms_r16_inplace(v[m], nullptr, 256);
        uint16_t* kd = KCl + (size_t)(p0 + m) * 256;
        uint16_t* vd = VCl + (size_t)(p0 + m) * 256;
        for (int i = 0; i < 256; i += 8) {
          _mm_storeu_si128((__m128i*)(kd + i), f2bf8(_mm256_loadu_ps(k[m] + i)));
          _mm_storeu_si128((__m128i*)(vd + i), f2bf8(_mm256_loadu_ps(v[m] + i)));
        }
      }
      if (split) {  // E:1325-1327
        AttnArg aa;
        aa.Kc = KCl;
        aa.Vc = VCl;
        aa.hd = 256;
        aa.nh = 8;
        aa.M = M;
        aa.kmax = p0 + M - 1;
        aa.kmin = aa.kmax;
        float* outp[4];
        for (int m = 0; m < M; ++m) {
          aa.q[m] = q[m];
          aa.pos[m] = p0 + m;
          aa.lo[m] = A.sliding ? std::max(0, p0 + m - 511) : 0;
          aa.skip_lo[m] = 1;
          aa.skip_hi[m] = 0;
          aa.kmin = std::min(aa.kmin, aa.lo[m]);
          outp[m] = att[m];
        }
        POOL.run(attn_task, &aa);
        attn_merge(aa, T, outp, nullptr);
      } else if (tiled) {
        ref_attn_tile(KCl, VCl, A.sliding, &q[0][0], p0, M, &att[0][0]);
      } else {
        run_mh_rows(KCl, VCl, A.sliding, &q[0][0], p0, M, &att[0][0]);
      }
      XB.prep(&att[0][0], 2048, M);
      lin1(XB, qm[3], &o[0][0]);  // E:1356
      for (int m = 0; m < M; ++m) {  // E:1358-1361
        rbf_n(o[m], H);
        rms(o[m], A.nv[1], H, tmp);
        add_res_inplace(x[m], tmp, H);
        rms_prep_x(x[m], A.nv[2], H, mlp_in[m], XA.xe + (size_t)m * (H / 2), XA.xo + (size_t)m * (H / 2),
                   XA.gs + (size_t)m * (H / 32), true);
      }
      XA.K = H;
      XA.M = M;
      XA.src = &mlp_in[0][0];
      XA.qdone = false;
      if (G_I8_ACTIVE && M >= 2) {  // E:1367-1371
        const Q4* qq[2] = {&qm[4], &qm[5]};
        float* yy[2] = {gbuf.data(), ubuf.data()};
        lin_multi(XA, 2, qq, yy);
        for (int m = 0; m < M; ++m) {
          const float* gm = gbuf.data() + (size_t)m * I;
          const float* um = ubuf.data() + (size_t)m * I;
          float* am = abuf.data() + (size_t)m * I;
          for (int i = 0; i < I; i += 8) {
            __m256 g = rbf8(_mm256_loadu_ps(gm + i)), u = rbf8(_mm256_loadu_ps(um + i));
            _mm256_storeu_ps(am + i, rbf8(_mm256_mul_ps(rbf8(gelu8(g)), u)));
          }
        }
        XB.prep(abuf.data(), I, M);
      } else {  // E:1363-1366
        XB.K = I;
        XB.M = M;
        XB.src = abuf.data();
        XB.qdone = false;
        GateUpArg gua{&XA, &qm[4], &qm[5], gbuf.data(), ubuf.data(), abuf.data(), &XB};
        POOL.run(gate_up_fused_task, &gua);
      }
      lin1(XB, qm[6], &o[0][0]);  // E:1373
      const __m256 vsc = _mm256_set1_ps(A.scalar);
      for (int m = 0; m < M; ++m) {  // E:1375-1404, zero per-layer-embedding branch
        rbf_n(o[m], H);
        rms(o[m], A.nv[3], H, tmp);
        add_res_prep_x(x[m], tmp, H, XA.xe + (size_t)m * (H / 2), XA.xo + (size_t)m * (H / 2), XA.gs + (size_t)m * (H / 32));
        for (int i = 0; i < H; i += 8) _mm256_storeu_ps(x[m] + i, rbf8(_mm256_mul_ps(_mm256_loadu_ps(x[m] + i), vsc)));
        if (l + 1 < NL)
          rms_prep_x(x[m], md->L[l + 1].nv[0], H, a[m], XA.xe + (size_t)m * (H / 2), XA.xo + (size_t)m * (H / 2),
                     XA.gs + (size_t)m * (H / 32), false);
        else if (last && m == M - 1 && hlast) {
          rms(x[m], md->fnorm, H, hlast);
          rbf_n(hlast, H);
        }
      }
      XA.K = H;
      XA.M = M;
      XA.src = &a[0][0];
      XA.qdone = false;
    }
    done += M;
  }
  G_I8_ACTIVE = false;
  return 0;
}


// ---------------------------------------------------------------------------------------
// MTP drafter step (E:1534-1563) on a synthetic drafter: the engine's b16_rows (through
// b16_multi), d_gate_up_task, dcand_task, attn_task + attn_merge, rms, rms_r16_inplace,
// rope_avx2, composed as draft_step does; the top-32 and best / second-best scans restate the
// lambda's lines.  Tensors come from the oracle's drafter (g4o_drafter_ptr names).
// ---------------------------------------------------------------------------------------
struct RefDrafter {
  const uint16_t *pre, *post, *cent, *emb;
  const uint16_t *q[4], *o[4], *gate[4], *up[4], *down[4];
  const float* nv[4][5];
  const float* dnorm;
  const int64_t* order;
  int C;
};

void ref_b16(const uint16_t* W, int N, int K, const float* x, float* y) {
  B16 m{W, N, K};
  b16_1(x, m, y);
}

int ref_draft_step(RefModel* md, const RefDrafter* d, int tok, const float* h, int pos, int P, int T, float* b_out,
                   int* sec_out, float* gap_out) {
  const int H = 1536;
  if (T < 1 || T > 16 || md->NL < 15) return -1;
  alignas(32) static float dcomb[3072], dx[256], da[256], dq[1024], dopt[1024], dtmp[256], dgate[2048], dup[2048],
      dact[2048], dh[256];
  static std::vector<float> dscore;
  static int cand[4096];
  static float cscore[4096];
  dscore.resize(d->C);
  G_I8_ACTIVE = false;
  const __m256 vsqh = _mm256_set1_ps(sqrtf((float)H));
  const uint16_t* er = md->E + (size_t)tok * H;
  for (int i = 0; i < H; i += 8) _mm256_storeu_ps(dcomb + i, rbf8(_mm256_mul_ps(bf8(er + i), vsqh)));
  std::memcpy(dcomb + H, h, H * 4);
  b16_1(dcomb, B16{d->pre, 256, 3072}, dx);
  rbf_n(dx, 256);
  for (int l = 0; l < 4; ++l) {
    const int hd = 256, ty = l < 3 ? 0 : 1, ol = l < 3 ? 13 : 14;
    const float* cs = md->cs[ty] + (size_t)pos * hd / 2;
    const float* sn = md->sn[ty] + (size_t)pos * hd / 2;
    rms(dx, d->nv[l][0], 256, da);
    b16_1(da, B16{d->q[l], 1024, 256}, dq);
    for (int h2 = 0; h2 < 4; ++h2) {
      float* qh = dq + h2 * hd;
      rms_r16_inplace(qh, d->nv[l][4], hd);
      rope_avx2(qh, cs, sn, hd);
    }
    {
      AttnArg aa;
      aa.Kc = md->KC + (size_t)ol * md->ctx * 256;
      aa.Vc = md->VC + (size_t)ol * md->ctx * 256;
      aa.hd = hd;
      aa.nh = 4;
      aa.M = 1;
      aa.q[0] = dq;
      aa.pos[0] = P;
      aa.skip_lo[0] = 1;
      aa.skip_hi[0] = 0;
      aa.lo[0] = l < 3 ? std::max(0, pos - 511) : 0;
      aa.kmin = aa.lo[0];
      aa.kmax = P;
      float* outp[1] = {dopt};
      for (int t = 0; t < T; ++t) attn_task(&aa, t, T);
      attn_merge(aa, T, outp);
    }
    b16_1(dopt, B16{d->o[l], 256, 1024}, da);
    rbf_n(da, 256);
    rms(da, d->nv[l][1], 256, dtmp);
    add_res_inplace(dx, dtmp, 256);
    rms(dx, d->nv[l][2], 256, da);
    rbf_n(da, 256);
    {
      B16 gm{d->gate[l], 2048, 256}, um{d->up[l], 2048, 256};
      DGateUpArg dgua{da, &gm, &um, dgate, dup, dact};
      POOL.run(d_gate_up_task, &dgua);
    }
    b16_1(dact, B16{d->down[l], 256, 2048}, da);
    rbf_n(da, 256);
    rms(da, d->nv[l][3], 256, dtmp);
    add_res_inplace(dx, dtmp, 256);
    const __m256 vdsc = _mm256_set1_ps(0.75f);
    for (int i = 0; i < 256; i += 8) _mm256_storeu_ps(dx + i, rbf8(_mm256_mul_ps(_mm256_loadu_ps(dx + i), vdsc)));
  }
  rms(dx, d->dnorm, 256, dh);
  rbf_n(dh, 256);
  {
    B16 pm{d->post, 1536, 256}, cm{d->cent, d->C, 256};
    const B16* mm[2] = {&pm, &cm};
    float* yy[2] = {b_out, dscore.data()};
    b16_multi(dh, 2, mm, yy);
  }
  rbf_n(b_out, H);
  int top[32];
  {
    float thr[32];
    int cnt = 0;
    for (int c = 0; c < d->C; ++c) {
      float s = dscore[c];
      if (cnt < 32) {
        int j = cnt++;
        while (j > 0 && thr[j - 1] < s) {
          thr[j] = thr[j - 1];
          top[j] = top[j - 1];
          --j;
        }
        thr[j] = s;
        top[j] = c;
      } else if (s > thr[31]) {
        int j = 31;
        while (j > 0 && thr[j - 1] < s) {
          thr[j] = thr[j - 1];
          top[j] = top[j - 1];
          --j;
        }
        thr[j] = s;
        top[j] = c;
      }
    }
  }
  int nc = 0;
  for (int t = 0; t < 32; ++t)
    for (int j = 0; j < 128; ++j) cand[nc++] = (int)d->order[(size_t)top[t] * 128 + j];
  {
    DCandArg dca{d->emb, cand, dh, cscore, nc};
    POOL.run(dcand_task, &dca);
  }
  int bestc = cand[0];
  float bs = -1e30f, bs2 = -1e30f;
  int sec = -1;
  for (int ci = 0; ci < nc; ++ci) {
    float sc2 = cscore[ci];
    if (sc2 > bs) {
      bs2 = bs;
      sec = bestc;
      bs = sc2;
      bestc = cand[ci];
    } else if (sc2 > bs2) {
      bs2 = sc2;
      sec = cand[ci];
    }
  }
  if (sec_out) *sec_out = sec;
  if (gap_out) *gap_out = bs - bs2;
  return bestc;
}

int ref_verify_ex(RefModel* md, const int* toks, int na, int nb, int pos0, int allow_b, RefOut* out);
// the final-normed hidden state of the last verify pass's last committed row (the next draft
// chain starts from it)
static float g_last_hidden[1536];
void ref_last_hidden(float* out) { std::memcpy(out, g_last_hidden, sizeof g_last_hidden); }
int ref_verify(RefModel* md, const int* toks, int na, int nb, int pos0, RefOut* out) {
  return ref_verify_ex(md, toks, na, nb, pos0, 1, out);
}
// allow_b = 0: branch b is never committed (E:1650 when the sibling's tree hit is not taken)
int ref_verify_ex(RefModel* md, const int* toks, int na, int nb, int pos0, int allow_b, RefOut* out) {
  const int H = 1536, M = 1 + na + nb, NL = md->NL, I = md->I;
  if (M > 8 || md->V != 262144) return -1;
  const int T = POOL.active_count();
  G_I8_ACTIVE = false;
  alignas(64) static float x[8][1536], q[8][2048], k[8][256], v[8][256], att[8][2048], o[8][1536], tmp[1536],
      hbuf[8][1536];
  static std::vector<float> gbuf, ubuf, abuf;
  gbuf.resize((size_t)8 * I);
  ubuf.resize((size_t)8 * I);
  abuf.resize((size_t)8 * I);
  static XP XA, XB;
  int rope[8], skl[8], skh[8];
  for (int r = 0; r < M; ++r) {
    if (r <= na) {
      rope[r] = pos0 + r;
      skl[r] = 1;
      skh[r] = 0;
    } else {
      rope[r] = pos0 + (r - na);
      skl[r] = pos0 + 1;
      skh[r] = pos0 + na;
    }
  }
  const __m256 vsqh = _mm256_set1_ps(sqrtf((float)H));
  for (int m = 0; m < M; ++m) {  // E:1262-1267
    const uint16_t* er = md->E + (size_t)toks[m] * H;
    for (int i = 0; i < H; i += 8) _mm256_storeu_ps(x[m] + i, rbf8(_mm256_mul_ps(bf8(er + i), vsqh)));
    rms_prep_x(x[m], md->L[0].nv[0], H, nullptr, XA.xe + (size_t)m * (H / 2), XA.xo + (size_t)m * (H / 2),
               XA.gs + (size_t)m * (H / 32), false);
  }
  XA.K = H;
  XA.M = M;
  for (int l = 0; l < NL; ++l) {
    const RefLayer& A = md->L[l];
    Q4 qm[7];
    const int Ns[7] = {2048, 256, 256, 1536, I, I, 1536}, Ks[7] = {1536, 1536, 1536, 2048, 1536, 1536, I};
    for (int j = 0; j < 7; ++j) {
      qm[j].w = A.W[j];
      qm[j].s = A.S[j];
      qm[j].N = Ns[j];
      qm[j].K = Ks[j];
    }
    {  // E:1289
      const Q4* qq[3] = {&qm[0], &qm[1], &qm[2]};
      float* yy[3] = {&q[0][0], &k[0][0], &v[0][0]};
      lin_multi(XA, 3, qq, yy);
    }
    const int ty = A.sliding ? 0 : 1;
    uint16_t* KCl = md->KC + (size_t)l * md->ctx * 256;
    uint16_t* VCl = md->VC + (size_t)l * md->ctx * 256;
    for (int m = 0; m < M; ++m) {  // E:1307-1324
      const float* cs = md->cs[ty] + (size_t)rope[m] * 128;
      const float* sn = md->sn[ty] + (size_t)rope[m] * 128;
      for (int h = 0; h < 8; ++h) {
        rms_r16_inplace(q[m] + h * 256, A.nv[4], 256);
        rope_avx2(q[m] + h * 256, cs, sn, 256);
      }
      rms_r16_inplace(k[m], A.nv[5], 256);
      rope_avx2(k[m], cs, sn, 256);
      rms_r16_inplace(v[m], nullptr, 256);
      uint16_t* kd = KCl + (size_t)(pos0 + m) * 256;
      uint16_t* vd = VCl + (size_t)(pos0 + m) * 256;
      for (int i = 0; i < 256; i += 8) {
        _mm_storeu_si128((__m128i*)(kd + i), f2bf8(_mm256_loadu_ps(k[m] + i)));
        _mm_storeu_si128((__m128i*)(vd + i), f2bf8(_mm256_loadu_ps(v[m] + i)));
      }
    }
    int lo[8], kmax = pos0 + M - 1, kmin = kmax;  // E:1325-1326
    for (int m = 0; m < M; ++m) {
      lo[m] = A.sliding ? std::max(0, rope[m] - 511) : 0;
      kmin = std::min(kmin, lo[m]);
    }
    // E:1305 / 1328 / 1337 (SPLITKV, TILED, ATT_PAR = 192): a chain pass, or the engine's sibling
    // form (one branch row, at most 4 rows; no attn_tile with a sibling); larger trees (the
    // generalisation the engine does not form) keep the split path
    const int sibling = (nb == 1 && M <= 4) ? na + 1 : -1;
    const bool split = nb > 1 || (nb == 1 && M > 4) || (M <= 4 && pos0 + M > 192);
    if (!split && nb == 0 && M >= 4 && pos0 + M > 64) ref_attn_tile(KCl, VCl, A.sliding, &q[0][0], pos0, M, &att[0][0]);
    else if (!split) run_mh_rows(KCl, VCl, A.sliding, &q[0][0], pos0, M, &att[0][0], sibling);
    for (int g0 = 0; split && g0 < M; g0 += 4) {  // AttnArg holds 4 rows: same geometry, rows in groups
      AttnArg aa;
      aa.Kc = KCl;
      aa.Vc = VCl;
      aa.hd = 256;
      aa.nh = 8;
      aa.M = std::min(4, M - g0);
      aa.kmin = kmin;
      aa.kmax = kmax;
      float* outp[4];
      for (int mm = 0; mm < aa.M; ++mm) {
        const int m = g0 + mm;
        aa.q[mm] = q[m];
        aa.pos[mm] = pos0 + m;
        aa.lo[mm] = lo[m];
        aa.skip_lo[mm] = skl[m];
        aa.skip_hi[mm] = skh[m];
        outp[mm] = att[m];
      }
      POOL.run(attn_task, &aa);
      attn_merge(aa, T, outp, nullptr);
    }
    XB.prep(&att[0][0], 2048, M);
    lin1(XB, qm[3], &o[0][0]);  // E:1356
    for (int m = 0; m < M; ++m) {  // E:1358-1361
      rbf_n(o[m], H);
      rms(o[m], A.nv[1], H, tmp);
      add_res_inplace(x[m], tmp, H);
      rms_prep_x(x[m], A.nv[2], H, nullptr, XA.xe + (size_t)m * (H / 2), XA.xo + (size_t)m * (H / 2),
                 XA.gs + (size_t)m * (H / 32), true);
    }
    XA.K = H;
    XA.M = M;
    XB.K = I;
    XB.M = M;
    GateUpArg gua{&XA, &qm[4], &qm[5], gbuf.data(), ubuf.data(), abuf.data(), &XB};
    POOL.run(gate_up_fused_task, &gua);  // E:1366
    lin1(XB, qm[6], &o[0][0]);           // E:1373
    const __m256 vsc = _mm256_set1_ps(A.scalar);
    for (int m = 0; m < M; ++m) {  // E:1375-1404, zero per-layer-embedding branch
      rbf_n(o[m], H);
      rms(o[m], A.nv[3], H, tmp);
      add_res_prep_x(x[m], tmp, H, XA.xe + (size_t)m * (H / 2), XA.xo + (size_t)m * (H / 2), XA.gs + (size_t)m * (H / 32));
      for (int i = 0; i < H; i += 8) _mm256_storeu_ps(x[m] + i, rbf8(_mm256_mul_ps(_mm256_loadu_ps(x[m] + i), vsc)));
      if (l + 1 < NL)
        rms_prep_x(x[m], md->L[l + 1].nv[0], H, nullptr, XA.xe + (size_t)m * (H / 2), XA.xo + (size_t)m * (H / 2),
                   XA.gs + (size_t)m * (H / 32), false);
      else {
        rms(x[m], md->fnorm, H, hbuf[m]);
        rbf_n(hbuf[m], H);
      }
    }
    XA.K = H;
    XA.M = M;
  }
  int G[8], fb[8], ns[8];
  for (int r = 0; r < 8; ++r) G[r] = -1, fb[r] = 0, ns[r] = 0;
  const int sib = (nb == 1 && M <= 4) ? na + 1 : -1;
  for (int r0 = 0; r0 < M; r0 += 4) head_group_ref(hbuf, toks, M, r0, std::min(M, r0 + 4), r0 == 0, G, fb, ns, sib);
  // E:1647-1661 along the branch chosen by G[0]
  int path[8], np = 1, first = 0, len = 0, br = 0;
  path[0] = 0;
  if (na >= 1 && G[0] == toks[1]) {
    first = 1;
    len = na;
  } else if (allow_b && nb >= 1 && G[0] == toks[na + 1]) {
    first = na + 1;
    len = nb;
    br = 1;
  }
  for (int i = 0; i < len; ++i) {
    const int row = first + i;
    if (G[path[np - 1]] != toks[row] || G[row] < 0) break;
    path[np++] = row;
  }
  out->nacc = np - 1;
  out->branch = np > 1 ? br : 0;
  out->ncommit = np;
  std::memcpy(g_last_hidden, hbuf[path[np - 1]], sizeof g_last_hidden);  // E:1660 hprev = hbuf[nacc]
  for (int r = 0; r < 8; ++r) {
    out->commit[r] = r < np ? G[path[r]] : -1;
    out->G[r] = G[r];
    out->fallback[r] = fb[r];
    out->nsurv[r] = ns[r];
  }
  if (out->branch == 1)
    for (int l = 0; l < NL; ++l)
      for (int i = 1; i < np; ++i) {
        std::memcpy(md->KC + ((size_t)l * md->ctx + pos0 + i) * 256, md->KC + ((size_t)l * md->ctx + pos0 + path[i]) * 256, 512);
        std::memcpy(md->VC + ((size_t)l * md->ctx + pos0 + i) * 256, md->VC + ((size_t)l * md->ctx + pos0 + path[i]) * 256, 512);
      }
  return 0;
}

}  // extern "C"
