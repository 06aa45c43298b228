/* g4_oracle_gemma.c -- oracle for the Gemma-4-E2B layer layout (the checkpoint main() loads).
 *
 * TEST INFRASTRUCTURE (see g4_oracle.h).  Restates engine/gemma4_engine.cpp fwd (E:1256-1405)
 * in its exact-float form (ENGINE_PREFILL_INT8 unset, so G_I8_ACTIVE is false: every linear
 * layer is the W4G32 GEMV) for the layout of E:1222-1232:
 *   * layer l has head_dim 256 and a 512-position window when l % 5 != 4, else head_dim 512 and
 *     global attention (E:1225); q_proj has 8 * hd rows;
 *   * layers 0..14 own their KV (k_proj, v_proj, k_norm); layer l >= 15 reads the cache of
 *     layer 13 (sliding) or 14 (global) and computes no k / v (owner_of, E:1251, 1288, 1304);
 *   * the MLP width of a layer is its gate_proj row count (E:1363);
 *   * per-layer inputs: ple_fused_task (E:615-660) at the start of a pass, and per layer the
 *     gate (pg_fused_task, E:405-443), per_layer_projection, post_per_layer_input_norm and
 *     layer_scalar (E:1379-1404);
 *   * RoPE: sliding theta 1e4 with every frequency, global theta 1e6 with the first quarter
 *     (E:1246-1247).
 * Tensors are read in place through the pointers of g4o_gemma_in (a mapped checkpoint); the
 * per-layer embedding table is given as the rows of a list of token ids, the other rows being
 * zero.  The head (E:1406-1500) is g4o_model_head of a g4o_model built from the same embedding.
 */
#include "g4_oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define H 1536
#define NQ 8
#define PD 256
#define NLG 35
#define GMAXROWS 32 /* MM, E:178 */

struct g4o_gemma {
  g4o_gemma_in in;
  int ctx;
  float *nv[NLG][7]; /* in_ln, post_attn, pre_ff, post_ff, post_ple, qn, kn (kn: owners) */
  float scalar[NLG];
  float *plnorm, *fnorm;
  uint16_t *KC[15], *VC[15]; /* owners' caches [ctx][hd] */
  float *cs[2], *sn[2];
  int i8; /* G_I8_ACTIVE: the linear layers of blocks of M >= 2 rows run W4A8 (E:311) */
};

static float* widen(const uint16_t* b, int n) {
  float* f = (float*)malloc(sizeof(float) * n);
  for (int i = 0; i < n; ++i) f[i] = g4o_bf2f(b[i]);
  return f;
}

static int layer_hd(int l) { return l % 5 != 4 ? 256 : 512; }
static int owner_of(int l) { return l < 15 ? l : (l % 5 != 4 ? 13 : 14); } /* E:1251 */

g4o_gemma* g4o_gemma_new(const g4o_gemma_in* in, int ctx) {
  g4o_gemma* g = (g4o_gemma*)calloc(1, sizeof(g4o_gemma));
  g->in = *in;
  g->ctx = ctx;
  for (int l = 0; l < NLG; ++l) {
    const g4o_glayer_in* A = &in->L[l];
    const int hd = layer_hd(l);
    g->nv[l][0] = widen(A->in_ln, H);
    g->nv[l][1] = widen(A->post_attn, H);
    g->nv[l][2] = widen(A->pre_ff, H);
    g->nv[l][3] = widen(A->post_ff, H);
    g->nv[l][4] = widen(A->post_ple, H);
    g->nv[l][5] = widen(A->qn, hd);
    g->nv[l][6] = l < 15 ? widen(A->kn, hd) : NULL;
    g->scalar[l] = g4o_bf2f(A->scalar);
  }
  g->plnorm = widen(in->plnorm, PD);
  g->fnorm = widen(in->fnorm, H);
  for (int l = 0; l < 15; ++l) {
    g->KC[l] = (uint16_t*)calloc((size_t)ctx * layer_hd(l), 2);
    g->VC[l] = (uint16_t*)calloc((size_t)ctx * layer_hd(l), 2);
  }
  for (int ty = 0; ty < 2; ++ty) { /* E:1246-1247 */
    const int hd = ty ? 512 : 256;
    g->cs[ty] = (float*)malloc(sizeof(float) * (size_t)ctx * hd / 2);
    g->sn[ty] = (float*)malloc(sizeof(float) * (size_t)ctx * hd / 2);
    g4o_rope_tables(ctx, hd, ty ? 1e6 : 1e4, ty ? 0.25 : 1.0, g->cs[ty], g->sn[ty]);
  }
  return g;
}

void g4o_gemma_free(g4o_gemma* g) {
  if (!g) return;
  for (int l = 0; l < NLG; ++l)
    for (int t = 0; t < 7; ++t) free(g->nv[l][t]);
  free(g->plnorm);
  free(g->fnorm);
  for (int l = 0; l < 15; ++l) {
    free(g->KC[l]);
    free(g->VC[l]);
  }
  for (int ty = 0; ty < 2; ++ty) {
    free(g->cs[ty]);
    free(g->sn[ty]);
  }
  free(g);
}

/* what the drafter reads of the target (E:1537, 1540-1543): the embedding, owner caches 13 and
 * 14, and the RoPE tables of both layer types */
void g4o_gemma_target(const g4o_gemma* g, const uint16_t** E, const uint16_t** K, const uint16_t** V,
                      const float** cs, const float** sn, int* hd) {
  *E = g->in.E;
  for (int ty = 0; ty < 2; ++ty) {
    K[ty] = g->KC[13 + ty];
    V[ty] = g->VC[13 + ty];
    cs[ty] = g->cs[ty];
    sn[ty] = g->sn[ty];
    hd[ty] = ty ? 512 : 256;
  }
}

/* E:1651: the KV rows of slot `from` copied to slot `to` in every owner cache */
void g4o_gemma_kv_move(g4o_gemma* g, int from, int to) {
  for (int l = 0; l < 15; ++l) {
    const int hd = layer_hd(l);
    memcpy(g->KC[l] + (size_t)to * hd, g->KC[l] + (size_t)from * hd, sizeof(uint16_t) * hd);
    memcpy(g->VC[l] + (size_t)to * hd, g->VC[l] + (size_t)from * hd, sizeof(uint16_t) * hd);
  }
}

const uint16_t* g4o_gemma_cache(const g4o_gemma* g, int l, int v) {
  if (l < 0 || l >= 15) return NULL;
  return v ? g->VC[l] : g->KC[l];
}

/* lin_multi (E:310-318): W4A8 for blocks of two rows or more while prompt blocks run int8 --
 * every matrix of the layout has its int8 tiles then (E:175, E:1505-1507), the per-layer-input
 * ones included (E:1270, E:1382-1385) -- else the exact W4G32 product */
static void gemv(int i8, const g4o_q4* q, const float* X, int M, float* Y) {
  if (i8 && M >= 2) g4o_w4a8_gemm(q->w, q->s, X, M, q->N, q->K, Y);
  else g4o_w4g32_gemm(q->w, q->s, X, M, q->N, q->K, Y);
}

void g4o_gemma_set_i8(g4o_gemma* g, int on) { g->i8 = on != 0; }

/* the token's row of the per-layer embedding table (zero for ids not listed) */
static const uint16_t* ple_row(const g4o_gemma* g, int tok) {
  int lo = 0, hi = g->in.nple - 1;
  while (lo <= hi) {
    const int mid = (lo + hi) / 2;
    if (g->in.ple_ids[mid] == tok) return g->in.ple_rows + (size_t)mid * NLG * PD;
    if (g->in.ple_ids[mid] < tok) lo = mid + 1;
    else hi = mid - 1;
  }
  return NULL;
}

/* fwd (E:1256-1405) of M <= 32 rows toks at positions pos0.. with T attention splits (the pool's
 * active workers) and the sibling row index (-1: none, E:1292, 1309, 1326, 1340-1345).
 * hbuf (optional) receives r16(rms(x, fnorm)) of rows m >= hf (E:1398-1400). */
void g4o_gemma_forward(g4o_gemma* g, const int* toks, int M, int pos0, int T, int sibling, float* hbuf, int hf) {
  if (M < 1 || M > GMAXROWS) return;
  const g4o_gemma_in* in = &g->in;
  float* x = (float*)malloc(sizeof(float) * M * H);
  float* xa = (float*)malloc(sizeof(float) * M * H);
  float* pr = (float*)malloc(sizeof(float) * M * NLG * PD);
  float* pli = (float*)malloc(sizeof(float) * M * NLG * PD);
  float* q = (float*)malloc(sizeof(float) * M * NQ * 512);
  float* k = (float*)malloc(sizeof(float) * M * 512);
  float* v = (float*)malloc(sizeof(float) * M * 512);
  float* att = (float*)malloc(sizeof(float) * M * NQ * 512);
  float* o = (float*)malloc(sizeof(float) * M * H);
  float* tmp = (float*)malloc(sizeof(float) * H);
  float* pgv = (float*)malloc(sizeof(float) * M * PD);
  float* g2 = (float*)malloc(sizeof(float) * M * PD);
  int Imax = 0;
  for (int l = 0; l < NLG; ++l) Imax = in->L[l].gate.N > Imax ? in->L[l].gate.N : Imax;
  float* gt = (float*)malloc(sizeof(float) * (size_t)M * Imax);
  float* up = (float*)malloc(sizeof(float) * (size_t)M * Imax);
  const float sqh = sqrtf((float)H);
  for (int m = 0; m < M; ++m) { /* E:1262-1267 */
    const uint16_t* er = in->E + (size_t)toks[m] * H;
    for (int c = 0; c < H; ++c) x[m * H + c] = g4o_r16(g4o_bf2f(er[c]) * sqh);
    g4o_rms(x + m * H, g->nv[0][0], H, xa + m * H);
  }
  /* E:615-660 ple_fused_task: per_layer_model_projection of the (un-normed) rows, then per
   * layer r16(. / sqrt(H)), rms over 256 with per_layer_projection_norm, plus r16(16 PLE row),
   * times 0.70710678118 */
  gemv(g->i8, &in->plproj, x, M, pr);
  const float s1 = 1.0f / sqrtf((float)H);
  for (int m = 0; m < M; ++m) {
    const uint16_t* pe = ple_row(g, toks[m]);
    for (int l = 0; l < NLG; ++l) {
      float* prl = pr + (size_t)m * NLG * PD + l * PD;
      float pj[PD];
      for (int i = 0; i < PD; ++i) prl[i] = g4o_r16(prl[i] * s1);
      g4o_rms(prl, g->plnorm, PD, pj);
      float* pl = pli + (size_t)m * NLG * PD + l * PD;
      for (int i = 0; i < PD; ++i) {
        const float pev = g4o_r16((pe ? g4o_bf2f(pe[l * PD + i]) : 0.0f) * 16.0f);
        pl[i] = (pj[i] + pev) * 0.70710678118f;
      }
    }
  }
  for (int l = 0; l < NLG; ++l) {
    const g4o_glayer_in* A = &in->L[l];
    const int hd = layer_hd(l), ty = l % 5 != 4 ? 0 : 1, sliding = ty == 0, own = l < 15, ol = owner_of(l);
    gemv(g->i8, &A->q, xa, M, q); /* E:1287-1288 */
    if (own) {
      gemv(g->i8, &A->k, xa, M, k);
      gemv(g->i8, &A->v, xa, M, v);
    }
    const int split = M <= 4 && pos0 + M > 192; /* E:1305 (ATT_PAR 192, SPLITKV) */
    const int tiled = !split && sibling < 0 && M >= 4 && pos0 + M > 64;
    int pos[GMAXROWS], lo[GMAXROWS], slo[GMAXROWS], shi[GMAXROWS], kmax = pos0 + M - 1, kmin = kmax;
    for (int m = 0; m < M; ++m) {
      const int cachepos = pos0 + m, rp = m == sibling ? pos0 + 1 : cachepos;
      const float* cs = g->cs[ty] + (size_t)rp * hd / 2;
      const float* sn = g->sn[ty] + (size_t)rp * hd / 2;
      for (int h = 0; h < NQ; ++h) { /* q norm + RoPE (E:1311-1312, 1331-1332, 1341-1342) */
        float* qh = q + (size_t)m * NQ * hd + h * hd;
        g4o_rms_r16_inplace(qh, g->nv[l][5], hd);
        g4o_rope(qh, cs, sn, hd);
      }
      if (own) { /* E:1290-1301, 1314-1321 */
        float* km = k + (size_t)m * hd;
        float* vm = v + (size_t)m * hd;
        g4o_rms_r16_inplace(km, g->nv[l][6], hd);
        g4o_rope(km, cs, sn, hd);
        g4o_rms_r16_inplace(vm, NULL, hd);
        uint16_t* kd = g->KC[l] + (size_t)cachepos * hd;
        uint16_t* vd = g->VC[l] + (size_t)cachepos * hd;
        for (int c = 0; c < hd; ++c) {
          kd[c] = g4o_f2bf(km[c]);
          vd[c] = g4o_f2bf(vm[c]);
        }
      }
      pos[m] = cachepos; /* E:1325-1326 */
      lo[m] = sliding ? (rp - 511 > 0 ? rp - 511 : 0) : 0;
      slo[m] = m == sibling ? pos0 + 1 : 1;
      shi[m] = m == sibling ? pos0 + m - 1 : 0;
      kmin = kmin < lo[m] ? kmin : lo[m];
    }
    const uint16_t* Kc = g->KC[ol];
    const uint16_t* Vc = g->VC[ol];
    if (split)
      g4o_attn_splitkv(Kc, Vc, hd, NQ, M, q, NQ * hd, pos, lo, slo, shi, kmin, kmax, T, att, NQ * hd, NULL, NULL);
    else if (tiled)
      g4o_attn_tile(Kc, Vc, hd, NQ, M, q, NQ * hd, pos, lo, att, NQ * hd); /* E:1328-1336 */
    else { /* run_mh (E:1337-1354): the sibling row skips the rows between row 0 and itself */
      int sl[GMAXROWS], sh[GMAXROWS];
      for (int m = 0; m < M; ++m) {
        sl[m] = m == sibling ? pos0 + 1 : 1;
        sh[m] = m == sibling ? pos0 + m - 1 : 0;
      }
      g4o_attn_mh(Kc, Vc, hd, NQ, M, q, NQ * hd, pos, lo, sl, sh, att, NQ * hd);
    }
    gemv(g->i8, &A->o, att, M, o); /* E:1356 */
    for (int m = 0; m < M; ++m) { /* E:1358-1361 */
      float* om = o + m * H;
      float* xm = x + m * H;
      for (int c = 0; c < H; ++c) om[c] = g4o_r16(om[c]);
      g4o_rms(om, g->nv[l][1], H, tmp);
      for (int c = 0; c < H; ++c) xm[c] = g4o_r16(xm[c] + g4o_r16(tmp[c]));
      g4o_rms(xm, g->nv[l][2], H, xa + m * H);
      for (int c = 0; c < H; ++c) xa[m * H + c] = g4o_r16(xa[m * H + c]);
    }
    const int I = A->gate.N; /* E:1363-1367, gate_up_fused_task (E:256-302) */
    gemv(g->i8, &A->gate, xa, M, gt);
    gemv(g->i8, &A->up, xa, M, up);
    for (size_t c = 0; c < (size_t)M * I; ++c) gt[c] = g4o_r16(g4o_r16(g4o_gelu8(g4o_r16(gt[c]))) * g4o_r16(up[c]));
    gemv(g->i8, &A->down, gt, M, o); /* E:1373 */
    for (int m = 0; m < M; ++m) { /* E:1375-1378: add_res_prep_x, the rows feed the gate as they are */
      float* om = o + m * H;
      float* xm = x + m * H;
      for (int c = 0; c < H; ++c) om[c] = g4o_r16(om[c]);
      g4o_rms(om, g->nv[l][3], H, tmp);
      for (int c = 0; c < H; ++c) xm[c] = g4o_r16(xm[c] + g4o_r16(tmp[c]));
    }
    gemv(g->i8, &A->pg, x, M, pgv); /* E:405-443 pg_fused_task */
    for (int m = 0; m < M; ++m) {
      const float* pl = pli + (size_t)m * NLG * PD + l * PD;
      for (int i = 0; i < PD; ++i)
        g2[m * PD + i] = g4o_r16(g4o_r16(g4o_gelu8(g4o_r16(pgv[m * PD + i]))) * g4o_r16(pl[i]));
    }
    gemv(g->i8, &A->pp, g2, M, o); /* E:1386 */
    for (int m = 0; m < M; ++m) { /* E:1387-1404 */
      float* om = o + m * H;
      float* xm = x + m * H;
      for (int c = 0; c < H; ++c) om[c] = g4o_r16(om[c]);
      g4o_rms(om, g->nv[l][4], H, tmp);
      for (int c = 0; c < H; ++c) xm[c] = g4o_r16(g4o_r16(xm[c] + g4o_r16(tmp[c])) * g->scalar[l]);
      if (l + 1 < NLG) g4o_rms(xm, g->nv[l + 1][0], H, xa + m * H);
      else if (hbuf && m >= hf) {
        g4o_rms(xm, g->fnorm, H, hbuf + m * H);
        for (int c = 0; c < H; ++c) hbuf[m * H + c] = g4o_r16(hbuf[m * H + c]);
      }
    }
  }
  free(x);
  free(xa);
  free(pr);
  free(pli);
  free(q);
  free(k);
  free(v);
  free(att);
  free(o);
  free(tmp);
  free(pgv);
  free(g2);
  free(gt);
  free(up);
}
