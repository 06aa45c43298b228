// ref_harness.cpp -- C entry points into the reference engine's own kernels.
//
// TEST INFRASTRUCTURE.  Built by oracle/Makefile from the reference sources where
// they lie (the engine is included with `#define main engine_main`, the trick the
// reference's bench/attn_bench.cpp:2-4 uses); the output goes to oracle/_ref/ only.
// Used to pin the C oracle bit-for-bit and as the "reference" CPU baseline.
// Every wrapper calls the reference's static functions unchanged; the few lines
// that compose them restate the call sites they cite (E = engine/gemma4_engine.cpp).
#define main engine_main
#include G4_REF_ENGINE
#undef main
#include <sched.h>

namespace {
XP g_xa, g_xb;
bool g_started = false;
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
  for (int i = 0; i < n; i += 8) _mm256_storeu_ps(y + i, exp8(_mm256_loadu_ps(x + i)));
}
void ref_gelu8(const float* x, int n, float* y) {
  for (int i = 0; i < n; i += 8) _mm256_storeu_ps(y + i, gelu8(_mm256_loadu_ps(x + i)));
}
void ref_rbf8(const float* x, int n, float* y) {
  for (int i = 0; i < n; i += 8) _mm256_storeu_ps(y + i, rbf8(_mm256_loadu_ps(x + i)));
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
void ref_attn(const uint16_t* Kc, const uint16_t* Vc, int hd, int nh, int M, const float* q, int ldq,
              const int* pos, const int* lo, const int* skip_lo, const int* skip_hi, int kmin,
              int kmax, int T, float* out, int ldo, float* xe, float* xo, float* gs, float* part_m,
              float* part_l) {
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

}  // extern "C"
