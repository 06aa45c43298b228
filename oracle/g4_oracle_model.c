/* g4_oracle_model.c -- oracle for the synthetic decoder stack and one tree verify pass.
 *
 * TEST INFRASTRUCTURE (see g4_oracle.h).  Restates the layer sequence of
 * engine/gemma4_engine.cpp fwd (E:1256-1405), the head (E:1406-1500) and the
 * acceptance/commit step (E:1647-1661) for the synthetic stack:
 *   * every layer owns its KV cache (no KV sharing), head_dim 256, 8 query heads,
 *     one KV head; layer l is sliding-window-512 when l % 5 != 4 (E:1225,1326);
 *   * the per-layer-embedding branch contributes zero, so the layer end
 *     rbf8(rbf8(x + rbf8(0)) * scalar) (E:1393) reduces to r16(x * scalar);
 *   * the draft tree is row 0 (confirmed token), chain a = rows 1..na at positions
 *     pos0+1.., and branch b = rows na+1..na+nb whose RoPE positions are pos0+1..
 *     while their cache slots follow chain a.  Branch rows skip chain a's slots;
 *     with nb = 1 this is exactly the reference's sibling row (E:1292,1309,1326).
 * Synthetic weights and the fake context are generated from seeds as documented
 * at g4o_model_new / g4o_model_fake_ctx.
 */
#include "g4_oracle.h"
#include "g4_rng.h"
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define H 1536
#define HD 256
#define NQ 8

typedef struct {
  uint8_t* W[7];
  uint16_t* S[7];
  int N[7], K[7];
  float* nv[6]; /* in_ln, post_attn, pre_ff, post_ff, qn, kn */
  float scalar;
  int sliding;
} olayer;

struct g4o_model {
  int V, NL, I, ctx;
  uint16_t* E;
  uint8_t* Wq;
  uint16_t* Sq;
  float* coef;
  uint8_t cb[8];
  uint8_t* x3;
  int64_t* xptr;
  uint16_t* xcol;
  float* xdel;
  olayer* L;
  float* fnorm;
  uint16_t *KC, *VC;            /* [NL][ctx][HD] */
  float *cs[2], *sn[2];         /* 0: sliding (theta 1e4, full rotary), 1: global (1e6, 0.25) */
};

/* Synthetic-stack generator (the product's generator implements the same formulas):
 *   E[n][k]      = f2bf(0.02 * normal(stream(seed, 1), n*H + k))
 *   W byte i     = (hash(stream(seed, 1000 + 10 l + j), i) >> 24) & 0xFF   (two uniform nibbles)
 *   S[i]         = f2bf(0.005 + 0.015 * unif(stream(seed, 2000 + 10 l + j), i))
 *   norm t, i    = r16(base_t + span_t * unif(stream(seed, 3000 + 10 l + t), i)),
 *                  (base, span) = (0.5, 1.0) for in_ln/post_attn/pre_ff/post_ff, (0.2, 0.1) for q/k norm
 *   scalar       = 0.75;  fnorm[i] = r16(0.5 + unif(stream(seed, 4000), i))
 * matrices j: 0 q [8*256 x H], 1 k [256 x H], 2 v [256 x H], 3 o [H x 8*256], 4 gate [I x H],
 *             5 up [I x H], 6 down [H x I]. */
static void gen_matrix(uint64_t seed, int l, int j, int N, int K, uint8_t* W, uint16_t* S) {
  uint64_t sw = g4r_stream(seed, 1000 + 10 * (uint64_t)l + j), ss = g4r_stream(seed, 2000 + 10 * (uint64_t)l + j);
  size_t nb = (size_t)N * K / 2, ns = (size_t)N * K / 32;
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < nb; ++i) W[i] = (uint8_t)((g4r_hash(sw, i) >> 24) & 0xFF);
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < ns; ++i) S[i] = g4o_f2bf(0.005f + 0.015f * g4r_unif(ss, i));
}

g4o_model* g4o_model_new(uint64_t seed, int V, int NL, int I, int ctx) {
  g4o_model* m = (g4o_model*)calloc(1, sizeof(g4o_model));
  m->V = V;
  m->NL = NL;
  m->I = I;
  m->ctx = ctx;
  m->E = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)V * H);
  uint64_t se = g4r_stream(seed, 1);
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < (size_t)V * H; ++i) m->E[i] = g4o_f2bf(0.02f * g4r_normal(se, i));
  m->L = (olayer*)calloc(NL, sizeof(olayer));
  const int Ns[7] = {NQ * HD, HD, HD, H, I, I, H}, Ks[7] = {H, H, H, NQ * HD, H, H, I};
  for (int l = 0; l < NL; ++l) {
    olayer* a = &m->L[l];
    for (int j = 0; j < 7; ++j) {
      a->N[j] = Ns[j];
      a->K[j] = Ks[j];
      a->W[j] = (uint8_t*)malloc((size_t)Ns[j] * Ks[j] / 2);
      a->S[j] = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)Ns[j] * Ks[j] / 32);
      gen_matrix(seed, l, j, Ns[j], Ks[j], a->W[j], a->S[j]);
    }
    for (int t = 0; t < 6; ++t) {
      int n = t < 4 ? H : HD;
      float base = t < 4 ? 0.5f : 0.2f, span = t < 4 ? 1.0f : 0.1f;
      uint64_t sn = g4r_stream(seed, 3000 + 10 * (uint64_t)l + t);
      a->nv[t] = (float*)malloc(sizeof(float) * n);
      for (int i = 0; i < n; ++i) a->nv[t][i] = g4o_r16(base + span * g4r_unif(sn, i));
    }
    a->scalar = 0.75f;
    a->sliding = (l % 5 != 4);
  }
  m->fnorm = (float*)malloc(sizeof(float) * H);
  uint64_t sf = g4r_stream(seed, 4000);
  for (int i = 0; i < H; ++i) m->fnorm[i] = g4o_r16(0.5f + g4r_unif(sf, i));
  /* head screen and exp3 head (E:1232-1244) */
  m->Wq = (uint8_t*)malloc((size_t)V * H / 2);
  m->Sq = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)V * H / 32);
  m->coef = (float*)malloc(sizeof(float) * V);
  g4o_screen_build(m->E, V, H, m->Wq, m->Sq, m->coef);
  g4o_exp3_codebook(m->E, (int64_t)V * H, m->cb);
  m->xptr = (int64_t*)malloc(sizeof(int64_t) * (V + 1));
  int64_t ne = g4o_exp3_count(m->E, V, H, m->cb, m->xptr);
  m->x3 = (uint8_t*)malloc((size_t)V * (H / 32) * 44);
  m->xcol = (uint16_t*)malloc(sizeof(uint16_t) * (ne + 1));
  m->xdel = (float*)malloc(sizeof(float) * (ne + 1));
  g4o_exp3_pack(m->E, V, H, m->cb, m->x3, m->xptr, m->xcol, m->xdel);
  m->KC = (uint16_t*)calloc((size_t)NL * ctx * HD, sizeof(uint16_t));
  m->VC = (uint16_t*)calloc((size_t)NL * ctx * HD, sizeof(uint16_t));
  for (int t = 0; t < 2; ++t) {
    m->cs[t] = (float*)malloc(sizeof(float) * (size_t)ctx * HD / 2);
    m->sn[t] = (float*)malloc(sizeof(float) * (size_t)ctx * HD / 2);
    g4o_rope_tables(ctx, HD, t ? 1e6 : 1e4, t ? 0.25 : 1.0, m->cs[t], m->sn[t]);
  }
  return m;
}

void g4o_model_free(g4o_model* m) {
  if (!m) return;
  free(m->E);
  free(m->Wq);
  free(m->Sq);
  free(m->coef);
  free(m->x3);
  free(m->xptr);
  free(m->xcol);
  free(m->xdel);
  for (int l = 0; l < m->NL; ++l) {
    for (int j = 0; j < 7; ++j) {
      free(m->L[l].W[j]);
      free(m->L[l].S[j]);
    }
    for (int t = 0; t < 6; ++t) free(m->L[l].nv[t]);
  }
  free(m->L);
  free(m->fnorm);
  free(m->KC);
  free(m->VC);
  for (int t = 0; t < 2; ++t) {
    free(m->cs[t]);
    free(m->sn[t]);
  }
  free(m);
}

/* E:1249-1250 ENGINE_FAKE_CTX: LCG rs = rs*1664525 + 1013904223 from `seed`, value
 * ((rs >> 9) % 2001 - 1000) / 700 rounded to bf16; layer by layer, K then V per element */
void g4o_model_fake_ctx(g4o_model* m, int n, uint64_t seed) {
  uint32_t rs = (uint32_t)seed;
  for (int l = 0; l < m->NL; ++l)
    for (size_t i = 0; i < (size_t)n * HD; ++i) {
      rs = rs * 1664525u + 1013904223u;
      m->KC[(size_t)l * m->ctx * HD + i] = g4o_f2bf((float)((int)(rs >> 9) % 2001 - 1000) / 700.0f);
      rs = rs * 1664525u + 1013904223u;
      m->VC[(size_t)l * m->ctx * HD + i] = g4o_f2bf((float)((int)(rs >> 9) % 2001 - 1000) / 700.0f);
    }
}

int g4o_model_ctx(const g4o_model* m) { return m->ctx; }

/* borrow a pointer to a named internal array (the reference harness runs on the same weights) */
const void* g4o_model_ptr(const g4o_model* m, const char* what) {
  int l = 0, j = 0;
  if (!strcmp(what, "E")) return m->E;
  if (!strcmp(what, "Wq")) return m->Wq;
  if (!strcmp(what, "Sq")) return m->Sq;
  if (!strcmp(what, "coef")) return m->coef;
  if (!strcmp(what, "cb")) return m->cb;
  if (!strcmp(what, "x3")) return m->x3;
  if (!strcmp(what, "xptr")) return m->xptr;
  if (!strcmp(what, "xcol")) return m->xcol;
  if (!strcmp(what, "xdel")) return m->xdel;
  if (!strcmp(what, "fnorm")) return m->fnorm;
  if (!strcmp(what, "KC")) return m->KC;
  if (!strcmp(what, "VC")) return m->VC;
  if (!strcmp(what, "cs0")) return m->cs[0];
  if (!strcmp(what, "sn0")) return m->sn[0];
  if (!strcmp(what, "cs1")) return m->cs[1];
  if (!strcmp(what, "sn1")) return m->sn[1];
  if (sscanf(what + 1, "%d_%d", &l, &j) == 2 && l >= 0 && l < m->NL) {
    if (what[0] == 'W' && j < 7) return m->L[l].W[j];
    if (what[0] == 'S' && j < 7) return m->L[l].S[j];
    if (what[0] == 'N' && j < 6) return m->L[l].nv[j];
  }
  return NULL;
}

/* copy a named internal array out (tests compare generated weights and caches) */
int g4o_model_bytes(const g4o_model* m, const char* what, void* dst, int64_t cap) {
  const void* src = NULL;
  int64_t nb = 0;
  if (!strcmp(what, "E")) { src = m->E; nb = (int64_t)m->V * H * 2; }
  else if (!strcmp(what, "Wq")) { src = m->Wq; nb = (int64_t)m->V * H / 2; }
  else if (!strcmp(what, "Sq")) { src = m->Sq; nb = (int64_t)m->V * H / 16; }
  else if (!strcmp(what, "coef")) { src = m->coef; nb = (int64_t)m->V * 4; }
  else if (!strcmp(what, "cb")) { src = m->cb; nb = 8; }
  else if (!strcmp(what, "xptr")) { src = m->xptr; nb = (int64_t)(m->V + 1) * 8; }
  else if (!strcmp(what, "KC")) { src = m->KC; nb = (int64_t)m->NL * m->ctx * HD * 2; }
  else if (!strcmp(what, "VC")) { src = m->VC; nb = (int64_t)m->NL * m->ctx * HD * 2; }
  else if (!strcmp(what, "fnorm")) { src = m->fnorm; nb = H * 4; }
  else if (!strncmp(what, "W", 1) || !strncmp(what, "S", 1) || !strncmp(what, "N", 1)) {
    int l = 0, j = 0;
    if (sscanf(what + 1, "%d_%d", &l, &j) != 2) return -1;
    if (l < 0 || l >= m->NL) return -1;
    if (what[0] == 'W' && j < 7) { src = m->L[l].W[j]; nb = (int64_t)m->L[l].N[j] * m->L[l].K[j] / 2; }
    else if (what[0] == 'S' && j < 7) { src = m->L[l].S[j]; nb = (int64_t)m->L[l].N[j] * m->L[l].K[j] / 16; }
    else if (what[0] == 'N' && j < 6) { src = m->L[l].nv[j]; nb = (j < 4 ? H : HD) * 4; }
  }
  if (!src || nb > cap) return -1;
  memcpy(dst, src, nb);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* forward                                                                  */
/* ------------------------------------------------------------------------ */

#define MAXROWS 32 /* MM, E:176: rows of one pass (prefill block) */
typedef struct {
  int M, pos0;
  int rope[MAXROWS], slot[MAXROWS], skip_lo[MAXROWS], skip_hi[MAXROWS];
} rows_t;

static void rows_tree(rows_t* r, int pos0, int na, int nb) {
  r->M = 1 + na + nb;
  r->pos0 = pos0;
  for (int i = 0; i < r->M; ++i) {
    r->slot[i] = pos0 + i;
    if (i <= na) {
      r->rope[i] = pos0 + i;
      r->skip_lo[i] = 1;
      r->skip_hi[i] = 0;
    } else {
      r->rope[i] = pos0 + (i - na);
      r->skip_lo[i] = pos0 + 1;
      r->skip_hi[i] = pos0 + na;
    }
  }
}

static void rows_chain(rows_t* r, int pos0, int M) {
  r->M = M;
  r->pos0 = pos0;
  for (int i = 0; i < M; ++i) {
    r->slot[i] = r->rope[i] = pos0 + i;
    r->skip_lo[i] = 1;
    r->skip_hi[i] = 0;
  }
}

/* attention path of a pass (E:1305, 1328, 1337) */
enum { ATT_SPLIT = 0, ATT_TILE = 1, ATT_MH = 2 };

/* a linear layer of the pass: lin_multi / lin1 (E:310-317) take W4A8 when G_I8_ACTIVE and the
 * pass has M >= 2 rows, else the exact-float W4G32 GEMV */
static void lin(int i8, const uint8_t* W, const uint16_t* S, const float* X, int M, int N, int K, float* Y) {
  if (i8 && M >= 2) g4o_w4a8_gemm(W, S, X, M, N, K, Y);
  else g4o_w4g32_gemm(W, S, X, M, N, K, Y);
}

/* E:1262-1405 for the rows r (M <= 32).  i8: G_I8_ACTIVE (prefill with ENGINE_PREFILL_INT8=1);
 * amode: the attention path.  hbuf (optional) receives r16(rms(x, fnorm)) of every row
 * (E:1400-1402). */
static void forward_ex(g4o_model* m, const int* toks, const rows_t* r, int T, float* hbuf, int i8, int amode) {
  const int M = r->M, I = m->I;
  float* x = (float*)malloc(sizeof(float) * M * H);
  float* xa = (float*)malloc(sizeof(float) * M * H);
  float* q = (float*)malloc(sizeof(float) * M * NQ * HD);
  float* k = (float*)malloc(sizeof(float) * M * HD);
  float* v = (float*)malloc(sizeof(float) * M * HD);
  float* att = (float*)malloc(sizeof(float) * M * NQ * HD);
  float* o = (float*)malloc(sizeof(float) * M * H);
  float* tmp = (float*)malloc(sizeof(float) * H);
  float* g = (float*)malloc(sizeof(float) * M * I);
  float* u = (float*)malloc(sizeof(float) * M * I);
  const float sqh = sqrtf((float)H);
  for (int i = 0; i < M; ++i) {
    const uint16_t* er = m->E + (size_t)toks[i] * H;
    for (int c = 0; c < H; ++c) x[i * H + c] = g4o_r16(g4o_bf2f(er[c]) * sqh); /* E:1265 */
    g4o_rms(x + i * H, m->L[0].nv[0], H, xa + i * H);                          /* E:1267 */
  }
  for (int l = 0; l < m->NL; ++l) {
    olayer* A = &m->L[l];
    const int ty = A->sliding ? 0 : 1;
    lin(i8, A->W[0], A->S[0], xa, M, A->N[0], H, q); /* E:1289 */
    lin(i8, A->W[1], A->S[1], xa, M, A->N[1], H, k);
    lin(i8, A->W[2], A->S[2], xa, M, A->N[2], H, v);
    int pos[MAXROWS], lo[MAXROWS], kmax = r->pos0 + M - 1, kmin = kmax;
    for (int i = 0; i < M; ++i) { /* E:1307-1324 */
      const float* cs = m->cs[ty] + (size_t)r->rope[i] * HD / 2;
      const float* sn = m->sn[ty] + (size_t)r->rope[i] * HD / 2;
      for (int h = 0; h < NQ; ++h) {
        g4o_rms_r16_inplace(q + (size_t)i * NQ * HD + h * HD, A->nv[4], HD);
        g4o_rope(q + (size_t)i * NQ * HD + h * HD, cs, sn, HD);
      }
      float* km = k + (size_t)i * HD;
      float* vm = v + (size_t)i * HD;
      g4o_rms_r16_inplace(km, A->nv[5], HD);
      g4o_rope(km, cs, sn, HD);
      g4o_rms_r16_inplace(vm, NULL, HD);
      uint16_t* kd = m->KC + ((size_t)l * m->ctx + r->slot[i]) * HD;
      uint16_t* vd = m->VC + ((size_t)l * m->ctx + r->slot[i]) * HD;
      for (int c = 0; c < HD; ++c) {
        kd[c] = g4o_f2bf(km[c]);
        vd[c] = g4o_f2bf(vm[c]);
      }
      pos[i] = r->slot[i]; /* E:1325-1326 */
      lo[i] = A->sliding ? (r->rope[i] - 511 > 0 ? r->rope[i] - 511 : 0) : 0;
      kmin = kmin < lo[i] ? kmin : lo[i];
    }
    const uint16_t* KCl = m->KC + (size_t)l * m->ctx * HD;
    const uint16_t* VCl = m->VC + (size_t)l * m->ctx * HD;
    if (amode == ATT_TILE) g4o_attn_tile(KCl, VCl, HD, NQ, M, q, NQ * HD, pos, lo, att, NQ * HD); /* E:1335 */
    else if (amode == ATT_MH) /* E:1337-1354, the sibling row's valid(p) (E:1345) as its skip range */
      g4o_attn_mh(KCl, VCl, HD, NQ, M, q, NQ * HD, pos, lo, r->skip_lo, r->skip_hi, att, NQ * HD);
    else
      g4o_attn_splitkv(KCl, VCl, HD, NQ, M, q, NQ * HD, pos, lo, r->skip_lo, r->skip_hi, kmin, kmax, T, att,
                       NQ * HD, NULL, NULL);
    lin(i8, A->W[3], A->S[3], att, M, H, NQ * HD, o); /* E:1356 */
    for (int i = 0; i < M; ++i) {                             /* E:1358-1361 */
      float* oi = o + i * H;
      float* xi = x + i * H;
      for (int c = 0; c < H; ++c) oi[c] = g4o_r16(oi[c]);
      g4o_rms(oi, A->nv[1], H, tmp);
      for (int c = 0; c < H; ++c) xi[c] = g4o_r16(xi[c] + g4o_r16(tmp[c]));
      g4o_rms(xi, A->nv[2], H, xa + i * H);
      for (int c = 0; c < H; ++c) xa[i * H + c] = g4o_r16(xa[i * H + c]);
    }
    lin(i8, A->W[4], A->S[4], xa, M, I, H, g); /* E:256-302 (i8: E:1368-1371) */
    lin(i8, A->W[5], A->S[5], xa, M, I, H, u);
    for (size_t c = 0; c < (size_t)M * I; ++c)
      g[c] = g4o_r16(g4o_r16(g4o_gelu8(g4o_r16(g[c]))) * g4o_r16(u[c]));
    lin(i8, A->W[6], A->S[6], g, M, H, I, o); /* E:1373 */
    for (int i = 0; i < M; ++i) {                     /* E:1375-1378, 1390-1404 */
      float* oi = o + i * H;
      float* xi = x + i * H;
      for (int c = 0; c < H; ++c) oi[c] = g4o_r16(oi[c]);
      g4o_rms(oi, A->nv[3], H, tmp);
      for (int c = 0; c < H; ++c) xi[c] = g4o_r16(xi[c] + g4o_r16(tmp[c]));
      for (int c = 0; c < H; ++c) xi[c] = g4o_r16(xi[c] * A->scalar);
      if (l + 1 < m->NL) g4o_rms(xi, m->L[l + 1].nv[0], H, xa + i * H);
      else if (hbuf) {
        g4o_rms(xi, m->fnorm, H, hbuf + i * H);
        for (int c = 0; c < H; ++c) hbuf[i * H + c] = g4o_r16(hbuf[i * H + c]);
      }
    }
  }
  free(x);
  free(xa);
  free(q);
  free(k);
  free(v);
  free(att);
  free(o);
  free(tmp);
  free(g);
  free(u);
}

/* the attention path of a decode pass of M rows at pos0 (E:1305, 1328, 1337 with SPLITKV, TILED,
 * ATT_PAR = 192): split-KV when M <= 4 and pos0 + M > 192, else attn_tile when M >= 4 and
 * pos0 + M > 64 and the pass has no sibling row, else run_mh.  A pass with one branch row and
 * at most 4 rows is the engine's sibling form (the branch row is `sibling`) and follows that
 * rule; larger trees (two branches of several rows, a generalisation the engine does not form)
 * keep the split-KV path for every size. */
static int pass_amode(int M, int pos0, int nb) {
  if (nb > 1 || (nb == 1 && M > 4)) return ATT_SPLIT;
  if (M <= 4 && pos0 + M > 192) return ATT_SPLIT;
  return (nb == 0 && M >= 4 && pos0 + M > 64) ? ATT_TILE : ATT_MH;
}

static void forward(g4o_model* m, const int* toks, const rows_t* r, int T, float* hbuf, int nb, int i8) {
  forward_ex(m, toks, r, T, hbuf, i8, pass_amode(r->M, r->pos0, nb));
}

/* E:1594-1599 prefill of toks[0..n) at positions pos0.. in blocks of pfb (<= 32) rows, with
 * ENGINE_PREFILL_INT8=1 (G_I8_ACTIVE during prefill, E:1595) and the engine's defaults
 * SPLITKV, TILED, ATT_PAR = 192 (E:1212-1214).  Per block of M rows at p0:
 *   attention: split-KV when M <= 4 and p0 + M > 192 (E:1305), else attn_tile when M >= 4 and
 *   p0 + M > 64 (E:1328), else run_mh (E:1337);  linear layers: W4A8 when M >= 2 (E:311).
 * hlast (optional) receives r16(rms(x, fnorm)) of the last row (E:1598, hf = M - 1). */
void g4o_prefill(g4o_model* m, const int* toks, int n, int pos0, int pfb, int T, float* hlast) {
  g4o_prefill_ex(m, toks, n, pos0, pfb, T, 1, hlast);
}

/* i8: G_I8 (ENGINE_PREFILL_INT8=1, E:1210): blocks of two rows or more multiply W4A8 (lin_multi,
 * E:311); 0: exact float throughout (the engine's default, G_I8 false) */
void g4o_prefill_ex(g4o_model* m, const int* toks, int n, int pos0, int pfb, int T, int i8, float* hlast) {
  if (pfb < 1) pfb = 1;
  if (pfb > MAXROWS) pfb = MAXROWS;
  float* hb = (float*)malloc(sizeof(float) * (size_t)MAXROWS * H);
  for (int done = 0; done < n;) {
    const int M = (n - done) < pfb ? (n - done) : pfb;
    const int p0 = pos0 + done;
    const int last = done + M == n;
    const int amode = (M <= 4 && p0 + M > 192) ? ATT_SPLIT : (M >= 4 && p0 + M > 64) ? ATT_TILE : ATT_MH;
    rows_t r;
    rows_chain(&r, p0, M);
    forward_ex(m, toks + done, &r, T, last ? hb : NULL, i8, amode);
    if (last && hlast) memcpy(hlast, hb + (size_t)(M - 1) * H, sizeof(float) * H);
    done += M;
  }
  free(hb);
}

void g4o_forward_fill(g4o_model* m, const int* toks, int M, int pos0, int T) {
  for (int b = 0; b < M; b += 8) {
    rows_t r;
    rows_chain(&r, pos0 + b, (M - b) < 8 ? (M - b) : 8);
    forward(m, toks + b, &r, T, NULL, 0, 0);
  }
}

static const int FIXED_SEEDS[20] = {2, 106, 107, 108, 235248, 235265, 235269, 476, 573, 577,
                                    604, 651, 688, 728, 785, 818, 947, 1024, 1154, 1280};

static void eval_row(g4o_model* m, const float* h, const int* toks, int M, g4o_verify_out* out,
                     int row) {
  int seeds[32], ns = 0;
  for (int i = 0; i < M && i < 8; ++i)
    if (toks[i] >= 0 && toks[i] < m->V) seeds[ns++] = toks[i]; /* E:1421 */
  for (int i = 0; i < 20; ++i) seeds[ns++] = FIXED_SEEDS[i];   /* E:1426 */
  int* surv = (int*)malloc(sizeof(int) * 30000);
  float* sval = (float*)malloc(sizeof(float) * 30000);
  g4o_head_info info;
  g4o_head_row(h, m->V, H, m->Wq, m->Sq, m->coef, m->x3, m->cb, m->xptr, m->xcol, m->xdel, seeds,
               ns, 30000, surv, sval, 30000, &info);
  out->G[row] = info.G;
  out->fallback[row] = info.fallback;
  out->nsurv[row] = info.nsurv;
  free(surv);
  free(sval);
}

/* the greedy token of one final-normed row h (E:1406-1500 for a single row, seeds: toks[0..nt)) */
int g4o_model_head(g4o_model* m, const float* h, const int* toks, int nt) {
  g4o_verify_out out;
  memset(&out, 0, sizeof out);
  eval_row(m, h, toks, nt, &out, 0);
  return out.G[0];
}

/* E:1453-1488 lazy head evaluation and E:1647-1661 acceptance, generalised to two branches:
 * branch a is walked when G[0] == toks[1]; otherwise branch b when G[0] == toks[b1]
 * (the reference's sibling test, E:1477).  Row r is evaluated only when the draft it holds
 * was accepted.  Branch b commits by copying its KV slots into place (E:1651). */
void g4o_verify(g4o_model* m, const int* toks, int na, int nb, int pos0, int T,
                g4o_verify_out* out, float* hidden_out) {
  g4o_verify_ex(m, toks, na, nb, pos0, T, 1, out, hidden_out);
}

/* allow_b = 0: branch b is never walked -- the engine's sibling row when its tree hit is not
 * taken (E:1650: neither TREE nor P + 1 + sibling <= ATT_PAR with gap1 >= 0.25), so acceptance
 * follows the chain alone (E:1656) */
void g4o_verify_ex(g4o_model* m, const int* toks, int na, int nb, int pos0, int T, int allow_b,
                   g4o_verify_out* out, float* hidden_out) {
  g4o_verify_i8(m, toks, na, nb, pos0, T, allow_b, 0, out, hidden_out);
}

/* i8: G_I8_ACTIVE in the decode (ENGINE_PREFILL_INT8=1 with ENGINE_DECODE_INT8 on, E:1600): the
 * pass's linear layers take W4A8 when it has two rows or more (lin, E:311) */
void g4o_verify_i8(g4o_model* m, const int* toks, int na, int nb, int pos0, int T, int allow_b, int i8,
                   g4o_verify_out* out, float* hidden_out) {
  rows_t r;
  rows_tree(&r, pos0, na, nb);
  const int M = r.M;
  float* hb = (float*)malloc(sizeof(float) * M * H);
  forward(m, toks, &r, T, hb, nb, i8);
  memset(out, 0, sizeof *out);
  for (int i = 0; i < 8; ++i) out->G[i] = -1;
  eval_row(m, hb, toks, M, out, 0);
  int path[8], np = 0, br = 0;
  path[np++] = 0;
  int first = -1, len = 0;
  if (na >= 1 && out->G[0] == toks[1]) {
    first = 1;
    len = na;
    br = 0;
  } else if (allow_b && nb >= 1 && out->G[0] == toks[na + 1]) {
    first = na + 1;
    len = nb;
    br = 1;
  }
  if (first > 0)
    for (int i = 0; i < len; ++i) {
      int row = first + i, prev = path[np - 1];
      if (out->G[prev] != toks[row]) break;
      eval_row(m, hb + (size_t)row * H, toks, M, out, row);
      path[np++] = row;
    }
  out->nacc = np - 1;
  out->branch = br;
  out->ncommit = np;
  for (int i = 0; i < np; ++i) out->commit[i] = out->G[path[i]];
  if (br == 1)
    for (int l = 0; l < m->NL; ++l)
      for (int i = 1; i < np; ++i) {
        size_t src = ((size_t)l * m->ctx + pos0 + path[i]) * HD, dst = ((size_t)l * m->ctx + pos0 + i) * HD;
        memcpy(m->KC + dst, m->KC + src, HD * 2);
        memcpy(m->VC + dst, m->VC + src, HD * 2);
      }
  if (hidden_out) memcpy(hidden_out, hb + (size_t)path[np - 1] * H, sizeof(float) * H);
  free(hb);
}
