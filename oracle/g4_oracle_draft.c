/* g4_oracle_draft.c -- oracle for the MTP drafter step (draft_step, E:1534-1563) on the synthetic
 * stack.
 *
 * TEST INFRASTRUCTURE (see g4_oracle.h).  Restates the drafter's layer sequence, its bf16
 * products (b16_rows, E:586-614), gate/up (d_gate_up_task, E:662-674), the centroid top-32
 * (E:1554-1555), candidate scoring (dcand_task, E:676-726) and the best / second-best scan
 * (E:1557-1559).  The drafter attends the target's KV cache of layer 13 (sliding layers) and
 * 14 (the global layer) with T splits (attn_task + attn_merge, E:1544-1545).
 *
 * g4o_drafter_load takes a drafter checkpoint's tensors instead (E:1519-1528: layer 3 of head
 * dim 512, layer scalars from the file), and g4o_gemma_draft_step runs a step against the
 * Gemma-4-E2B layout's owner caches 13 (head dim 256) and 14 (512).
 *
 * Synthetic drafter (the product's generator implements the same formulas): 4 layers of
 * hidden 256, 4 query heads of head_dim 256 (the reference's global drafter layer has
 * head_dim 512 like the target's layer 14; the synthetic target's layer 14 has 256), FFN 2048,
 * C = V / 128 centroids, every bf16 tensor f2bf(scale * normal(stream(seed, tag), i)):
 *   pre [256][3072] 0.02 (tag 5000); layer l: q [1024][256] 0.06 (5100+10l), o [256][1024] 0.03
 *   (5101+10l), gate [2048][256] 0.06 (5102+10l), up 0.06 (5103+10l), down [256][2048] 0.02
 *   (5104+10l); post [1536][256] 0.06 (5300), centroids [C][256] 0.06 (5301), token
 *   embedding [V][256] 0.06 (5303);
 *   norms r16(0.5 + unif) for in_ln, post_attn, pre_ff, post_ff (5200+10l+t, t = 0..3), final
 *   norm (5302); q norm r16(0.2 + 0.1 unif) (5204+10l); layer scalar 0.75;
 *   token order: Fisher-Yates over 0..V-1 with j = int(stream(seed, 5304), i, 0, i) for
 *   i = V-1 .. 1 (swap order[i], order[j]).
 */
#include "g4_oracle.h"
#include "g4_rng.h"
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define H 1536
#define DH 256
#define DQ 4
#define DF 2048

struct g4o_drafter {
  int V, C, owned; /* owned: the bf16 tensors were generated here (else they are the caller's) */
  int hd[4];       /* layer head dims: 256, and the global layer's (256 synthetic, 512 loaded) */
  float scalar[4];
  uint16_t *pre, *post, *cent, *emb;
  uint16_t *q[4], *o[4], *gate[4], *up[4], *down[4];
  float *nv[4][5]; /* in_ln, post_attn, pre_ff, post_ff, qn */
  float *dnorm;
  int64_t* order;
};

static uint16_t* gen_bf16(uint64_t seed, uint64_t tag, size_t n, float scale) {
  uint16_t* p = (uint16_t*)malloc(sizeof(uint16_t) * n);
  uint64_t s = g4r_stream(seed, tag);
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; ++i) p[i] = g4o_f2bf(scale * g4r_normal(s, i));
  return p;
}
static float* gen_norm(uint64_t seed, uint64_t tag, int n, float base, float span) {
  float* p = (float*)malloc(sizeof(float) * n);
  uint64_t s = g4r_stream(seed, tag);
  for (int i = 0; i < n; ++i) p[i] = g4o_r16(base + span * g4r_unif(s, i));
  return p;
}

g4o_drafter* g4o_drafter_new(uint64_t seed, int V) {
  g4o_drafter* d = (g4o_drafter*)calloc(1, sizeof(g4o_drafter));
  d->V = V;
  d->C = V / 128;
  d->owned = 1;
  for (int l = 0; l < 4; ++l) {
    d->hd[l] = DH;
    d->scalar[l] = 0.75f;
  }
  d->pre = gen_bf16(seed, 5000, (size_t)DH * 2 * H, 0.02f);
  for (int l = 0; l < 4; ++l) {
    d->q[l] = gen_bf16(seed, 5100 + 10 * l, (size_t)DQ * DH * DH, 0.06f);
    d->o[l] = gen_bf16(seed, 5101 + 10 * l, (size_t)DH * DQ * DH, 0.03f);
    d->gate[l] = gen_bf16(seed, 5102 + 10 * l, (size_t)DF * DH, 0.06f);
    d->up[l] = gen_bf16(seed, 5103 + 10 * l, (size_t)DF * DH, 0.06f);
    d->down[l] = gen_bf16(seed, 5104 + 10 * l, (size_t)DH * DF, 0.02f);
    for (int t = 0; t < 4; ++t) d->nv[l][t] = gen_norm(seed, 5200 + 10 * l + t, DH, 0.5f, 1.0f);
    d->nv[l][4] = gen_norm(seed, 5204 + 10 * l, DH, 0.2f, 0.1f);
  }
  d->post = gen_bf16(seed, 5300, (size_t)H * DH, 0.06f);
  d->cent = gen_bf16(seed, 5301, (size_t)d->C * DH, 0.06f);
  d->dnorm = gen_norm(seed, 5302, DH, 0.5f, 1.0f);
  d->emb = gen_bf16(seed, 5303, (size_t)V * DH, 0.06f);
  d->order = (int64_t*)malloc(sizeof(int64_t) * V);
  for (int i = 0; i < V; ++i) d->order[i] = i;
  uint64_t so = g4r_stream(seed, 5304);
  for (int i = V - 1; i >= 1; --i) {
    int j = g4r_int(so, (uint64_t)i, 0, i);
    int64_t t = d->order[i];
    d->order[i] = d->order[j];
    d->order[j] = t;
  }
  return d;
}

/* E:1519-1528: a drafter checkpoint's tensors (kept by the caller), norms widened here */
static float* widen_bf16(const uint16_t* b, int n) {
  float* f = (float*)malloc(sizeof(float) * n);
  for (int i = 0; i < n; ++i) f[i] = g4o_bf2f(b[i]);
  return f;
}

g4o_drafter* g4o_drafter_load(const g4o_drafter_in* in) {
  g4o_drafter* d = (g4o_drafter*)calloc(1, sizeof(g4o_drafter));
  d->V = in->V;
  d->C = in->C;
  d->owned = 0;
  d->pre = (uint16_t*)in->pre;
  d->post = (uint16_t*)in->post;
  d->cent = (uint16_t*)in->cent;
  d->emb = (uint16_t*)in->emb;
  d->order = (int64_t*)in->order;
  d->dnorm = widen_bf16(in->dnorm, DH);
  for (int l = 0; l < 4; ++l) {
    d->hd[l] = in->hd[l];
    d->scalar[l] = g4o_bf2f(in->scalar[l]);
    d->q[l] = (uint16_t*)in->q[l];
    d->o[l] = (uint16_t*)in->o[l];
    d->gate[l] = (uint16_t*)in->gate[l];
    d->up[l] = (uint16_t*)in->up[l];
    d->down[l] = (uint16_t*)in->down[l];
    for (int t = 0; t < 5; ++t) d->nv[l][t] = widen_bf16(in->nv[l][t], t < 4 ? DH : in->hd[l]);
  }
  return d;
}

void g4o_drafter_free(g4o_drafter* d) {
  if (!d) return;
  if (d->owned) {
    free(d->pre);
    free(d->post);
    free(d->cent);
    free(d->emb);
    free(d->order);
  }
  for (int l = 0; l < 4; ++l) {
    if (d->owned) {
      free(d->q[l]);
      free(d->o[l]);
      free(d->gate[l]);
      free(d->up[l]);
      free(d->down[l]);
    }
    for (int t = 0; t < 5; ++t) free(d->nv[l][t]);
  }
  free(d->dnorm);
  free(d);
}

const void* g4o_drafter_ptr(const g4o_drafter* d, const char* what) {
  int l = 0, t = 0;
  if (!strcmp(what, "pre")) return d->pre;
  if (!strcmp(what, "post")) return d->post;
  if (!strcmp(what, "cent")) return d->cent;
  if (!strcmp(what, "emb")) return d->emb;
  if (!strcmp(what, "dnorm")) return d->dnorm;
  if (!strcmp(what, "order")) return d->order;
  if (what[0] == 'L' && sscanf(what + 1, "%d_%d", &l, &t) == 2 && l >= 0 && l < 4) {
    switch (t) {
      case 0: return d->q[l];
      case 1: return d->o[l];
      case 2: return d->gate[l];
      case 3: return d->up[l];
      case 4: return d->down[l];
      default: break;
    }
    if (t >= 10 && t < 15) return d->nv[l][t - 10];
  }
  return NULL;
}

/* E:586-614 b16_rows: y[n] = hsum(a + b), a / b 8-lane FMA chains over k in steps of 16
 * (a: k = 16 s + l, b: k = 16 s + 8 + l) */
void g4o_b16_gemv(const uint16_t* W, int N, int K, const float* x, float* y) {
  for (int n = 0; n < N; ++n) {
    const uint16_t* w = W + (size_t)n * K;
    float a[8] = {0}, b[8] = {0}, v[8];
    for (int k = 0; k < K; k += 16)
      for (int l = 0; l < 8; ++l) {
        a[l] = fmaf(g4o_bf2f(w[k + l]), x[k + l], a[l]);
        b[l] = fmaf(g4o_bf2f(w[k + 8 + l]), x[k + 8 + l], b[l]);
      }
    for (int l = 0; l < 8; ++l) v[l] = a[l] + b[l];
    y[n] = ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
  }
}

static void r16n(float* p, int n) {
  for (int i = 0; i < n; ++i) p[i] = g4o_r16(p[i]);
}

/* the target as the drafter sees it: its embedding, the KV caches [ctx][hd] of layers 13
 * (type 0, the sliding drafter layers) and 14 (type 1, the global one) and the RoPE tables of
 * both types [ctx][hd / 2] */
typedef struct {
  const uint16_t* E;
  const uint16_t *K[2], *V[2];
  const float *cs[2], *sn[2];
  int hd[2];
} dr_target;

/* E:1534-1563 draft_step(tok, h, pos, P): the next draft token; b_out [1536] receives the
 * drafter's next hidden state, sec / gap the runner-up and the score gap (E:1559).  -1 when the
 * drafter's global layer and the target's layer 14 differ in head dim. */
static int draft_core(const dr_target* tg, const g4o_drafter* d, int tok, const float* h, int pos, int P, int T,
                      float* b_out, int* sec_out, float* gap_out) {
  if (d->hd[3] != tg->hd[1] || d->hd[0] != tg->hd[0]) return -1;
  float comb[2 * H], dx[DH], da[DH], dq[DQ * 512], dopt[DQ * 512], dtmp[DH], act[DF], g[DF], u[DF], dh[DH];
  const float sqh = sqrtf((float)H);
  for (int i = 0; i < H; ++i) comb[i] = g4o_r16(g4o_bf2f(tg->E[(size_t)tok * H + i]) * sqh); /* E:1537 */
  memcpy(comb + H, h, sizeof(float) * H);
  g4o_b16_gemv(d->pre, DH, 2 * H, comb, dx); /* E:1539 */
  r16n(dx, DH);
  for (int l = 0; l < 4; ++l) {
    const int sliding = l < 3, ty = sliding ? 0 : 1, hd = d->hd[l]; /* E:1540: layer 13 / 14 */
    const float* cs = tg->cs[ty] + (size_t)pos * hd / 2;
    const float* sn = tg->sn[ty] + (size_t)pos * hd / 2;
    g4o_rms(dx, d->nv[l][0], DH, da); /* E:1541 */
    g4o_b16_gemv(d->q[l], DQ * hd, DH, da, dq);
    for (int h2 = 0; h2 < DQ; ++h2) {
      g4o_rms_r16_inplace(dq + h2 * hd, d->nv[l][4], hd);
      g4o_rope(dq + h2 * hd, cs, sn, hd);
    }
    int apos = P, alo = sliding ? (pos - 511 > 0 ? pos - 511 : 0) : 0, sl = 1, sh = 0; /* E:1543 */
    g4o_attn_splitkv(tg->K[ty], tg->V[ty], hd, DQ, 1, dq, DQ * hd, &apos, &alo, &sl, &sh, alo, P, T, dopt, DQ * hd,
                     NULL, NULL);
    g4o_b16_gemv(d->o[l], DH, DQ * hd, dopt, da); /* E:1545 */
    r16n(da, DH);
    g4o_rms(da, d->nv[l][1], DH, dtmp);
    for (int i = 0; i < DH; ++i) dx[i] = g4o_r16(dx[i] + g4o_r16(dtmp[i]));
    g4o_rms(dx, d->nv[l][2], DH, da); /* E:1546 */
    r16n(da, DH);
    g4o_b16_gemv(d->gate[l], DF, DH, da, g); /* E:1547, d_gate_up_task E:662-674 */
    g4o_b16_gemv(d->up[l], DF, DH, da, u);
    for (int i = 0; i < DF; ++i) act[i] = g4o_r16(g4o_r16(g4o_gelu8(g4o_r16(g[i]))) * g4o_r16(u[i]));
    g4o_b16_gemv(d->down[l], DH, DF, act, da); /* E:1548 */
    r16n(da, DH);
    g4o_rms(da, d->nv[l][3], DH, dtmp);
    for (int i = 0; i < DH; ++i) dx[i] = g4o_r16(dx[i] + g4o_r16(dtmp[i]));
    for (int i = 0; i < DH; ++i) dx[i] = g4o_r16(dx[i] * d->scalar[l]); /* E:1549-1550 */
  }
  g4o_rms(dx, d->dnorm, DH, dh); /* E:1551 */
  r16n(dh, DH);
  float* dscore = (float*)malloc(sizeof(float) * d->C);
  g4o_b16_gemv(d->post, H, DH, dh, b_out); /* E:1552-1553 */
  g4o_b16_gemv(d->cent, d->C, DH, dh, dscore);
  r16n(b_out, H);
  int top[32];
  float thr[32];
  int cnt = 0;
  for (int c = 0; c < d->C; ++c) { /* E:1554-1555 */
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
  free(dscore);
  const int nc = cnt * 128;
  int bestc = 0, sec = -1;
  float bs = -1e30f, bs2 = -1e30f;
  for (int ci = 0; ci < nc; ++ci) { /* E:1556-1559 */
    const int cand = (int)d->order[(size_t)top[ci / 128] * 128 + ci % 128];
    float sc2;
    g4o_b16_gemv(d->emb + (size_t)cand * DH, 1, DH, dh, &sc2);
    if (ci == 0) bestc = cand;
    if (sc2 > bs) {
      bs2 = bs;
      sec = bestc;
      bs = sc2;
      bestc = cand;
    } else if (sc2 > bs2) {
      bs2 = sc2;
      sec = cand;
    }
  }
  if (sec_out) *sec_out = sec;
  if (gap_out) *gap_out = bs - bs2;
  return bestc;
}

/* m: the synthetic target (its embedding, RoPE tables and the KV cache of layers 13 and 14) */
int g4o_draft_step(const g4o_model* m, const g4o_drafter* d, int tok, const float* h, int pos, int P, int T,
                   float* b_out, int* sec_out, float* gap_out) {
  const uint16_t* KC = (const uint16_t*)g4o_model_ptr(m, "KC");
  const uint16_t* VC = (const uint16_t*)g4o_model_ptr(m, "VC");
  const size_t ctx = (size_t)g4o_model_ctx(m);
  dr_target t;
  t.E = (const uint16_t*)g4o_model_ptr(m, "E");
  for (int ty = 0; ty < 2; ++ty) {
    const int ol = 13 + ty;
    t.K[ty] = KC + ol * ctx * DH;
    t.V[ty] = VC + ol * ctx * DH;
    t.cs[ty] = (const float*)g4o_model_ptr(m, ty ? "cs1" : "cs0");
    t.sn[ty] = (const float*)g4o_model_ptr(m, ty ? "sn1" : "sn0");
    t.hd[ty] = DH;
  }
  return draft_core(&t, d, tok, h, pos, P, T, b_out, sec_out, gap_out);
}

/* g: the Gemma-4-E2B layout (owner caches 13 and 14 of head dim 256 / 512, E:1540) */
int g4o_gemma_draft_step(const g4o_gemma* g, const g4o_drafter* d, int tok, const float* h, int pos, int P, int T,
                         float* b_out, int* sec_out, float* gap_out) {
  dr_target t;
  g4o_gemma_target(g, &t.E, t.K, t.V, t.cs, t.sn, t.hd);
  return draft_core(&t, d, tok, h, pos, P, T, b_out, sec_out, gap_out);
}
