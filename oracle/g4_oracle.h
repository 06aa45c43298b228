/* g4_oracle.h -- CPU restatement of the reference's speculative-verify path.
 *
 * TEST INFRASTRUCTURE.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker (or as the
 * timed CPU baseline).  The product library never links it.
 *
 * Every function restates, in scalar C with explicit fmaf()/fma() calls, the
 * fp32 operation order of the reference function it cites
 * (dayaswaroopchavali/gemma4-e2b-laptop-cpu, files under engine/).  The file
 * is compiled with -ffp-contract=off so the compiler adds no contraction of
 * its own; every contraction that GCC performs in the reference build
 * (-O3 -march=x86-64-v3, default -ffp-contract=fast) is written out here.
 *
 * Pinning -- what checks each function (tests/test_golden.py against vectors written by
 * the reference's own kernels, tests/test_oracle_vs_ref.py against those kernels live,
 * tests/test_oracle_math.py against closed forms, bounds and brute force):
 *   f2bf/r16, exp8, gelu8, sumsq, rms*, rope   golden + live + fp64 / RNE brute force
 *   rope_tables                                fp64 closed form + the reference's main() (the
 *                                              Gemma-layout tokens and logit lines below use
 *                                              both tables)
 *   cap, calc_thr                              golden + live + defining property by scan
 *   prep_x, w4g32_*                            golden + live + fp64 closed form, row independence
 *   w4a8_quant, w4a8_gemm                      golden + live + exact integer part
 *   exp3_codebook                              most-frequent-exponent brute force only (the
 *                                              reference computes it inside main(), E:1232-1234)
 *   exp3_count/pack/dot/gemm                   golden (pack bytes, exceptions, logits) + round trip
 *   screen_build                               the screen main() builds (E:1235-1244), bit for
 *                                              bit, plus soundness and tightness of the bound
 *   head_row                                   golden survivor sets (reference scan) + screened
 *                                              greedy == brute-force full-head greedy
 *   attn_splitkv                               golden + live + fp64 softmax, LSE identity, masks
 *   attn_tile                                  live (the reference's attn_tile) + fp64 softmax
 *   attn_mh                                    fp64 softmax + the reference's main() through the
 *                                              Gemma-layout tokens and, per head row, its two
 *                                              largest logits printed by ENGINE_DEBUG_GAP (run_mh,
 *                                              E:1338-1349, is a lambda inside main())
 *   drafter (b16 gemv, draft step)             b16 gemv live against b16_rows; the step against
 *                                              the harness composition of the engine's kernels
 *   model / verify                             golden passes through the reference's kernels
 *                                              (2 layers, V 262144), acceptance brute force
 *   gemma (the Gemma-4-E2B layout)             FIRST / GEN tokens of the reference engine's main()
 *                                              run unchanged on the same synthetic checkpoint
 *                                              (tests/test_gemma_oracle.py), which change when
 *                                              the split count or the per-layer inputs do
 * Generators (g4_rng.h) are pinned by the CRC-32 of every input the fixtures store.
 */
#ifndef G4_ORACLE_H
#define G4_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar numerics (engine/gemma4_engine.cpp:33-60, 318-404) ---- */
uint16_t g4o_f2bf(float f);
float g4o_bf2f(uint16_t b);
float g4o_r16(float f);
float g4o_exp8(float x);
float g4o_gelu8(float x);
double g4o_sumsq(const float* x, int n);
float g4o_rms_inv(const float* x, int n);
void g4o_rms(const float* x, const float* w, int n, float* y);
void g4o_rms_r16_inplace(float* x, const float* w, int n);
void g4o_rope(float* h, const float* cs, const float* sn, int hd);
void g4o_rope_tables(int ctx, int hd, double theta, double rot_frac, float* cs, float* sn);
float g4o_cap(float s);
float g4o_calc_thr(float L);
void g4o_vec_exp8(const float* x, int n, float* y);
void g4o_vec_gelu8(const float* x, int n, float* y);

/* ---- W4G32 (engine/w4g32_avx2.h) ---- */
void g4o_prep_x(const float* x, int K, float* xe, float* xo, float* gs);
void g4o_w4g32_rows(const uint8_t* W, const uint16_t* S, const float* xe, const float* xo,
                    const float* gs, int K, int M, int n0, int n1, float* Y, int ldy);
void g4o_w4g32_gemm(const uint8_t* W, const uint16_t* S, const float* X, int M, int N, int K,
                    float* Y);

/* ---- prompt lookup (E:1624-1628): the most recent earlier occurrence of the last n tokens of
 * seq [L]; up to maxlen of the tokens that followed it go to drafts.  Returns their count. ---- */
int g4o_prompt_lookup(const int32_t* seq, int L, int n, int maxlen, int32_t* drafts);

/* ---- W4A8 (engine/w4a8_avx2.h) ---- */
void g4o_w4a8_quant(const float* X, int M, int K, int8_t* q, float* sx, int32_t* sum);
void g4o_w4a8_gemm(const uint8_t* W, const uint16_t* S, const float* X, int M, int N, int K,
                   float* Y);

/* ---- exp3-packed bf16 head (engine/bf16_exp3_head.h) ---- */
void g4o_exp3_codebook(const uint16_t* E, int64_t n, uint8_t cb8[8]);
int64_t g4o_exp3_count(const uint16_t* W, int N, int K, const uint8_t cb8[8], int64_t* exc_ptr);
void g4o_exp3_pack(const uint16_t* W, int N, int K, const uint8_t cb8[8], uint8_t* data,
                   const int64_t* exc_ptr, uint16_t* exc_col, float* exc_delta);
float g4o_exp3_dot(const uint8_t* data, const uint8_t cb8[8], const int64_t* exc_ptr,
                   const uint16_t* exc_col, const float* exc_delta, int K, int n, const float* x);
void g4o_exp3_gemm(const uint8_t* data, const uint8_t cb8[8], const int64_t* exc_ptr,
                   const uint16_t* exc_col, const float* exc_delta, int N, int K, const float* X,
                   int M, float* Y);

/* ---- certified head screen (engine/gemma4_engine.cpp:445-579, 1235-1244, 1409-1498) ---- */
void g4o_screen_build(const uint16_t* E, int N, int K, uint8_t* Wq, uint16_t* Sq, float* coef);

typedef struct {
  int G;            /* greedy token (lowest-index tie rule) */
  int fallback;     /* 1: full head was evaluated */
  int ref_overflow; /* 1: the reference's single-thread scan overflows its 16384 list */
  int nsurv;        /* survivors {U >= thr} (may exceed the limit) */
  float Lmax, thr, vmax;
} g4o_head_info;

/* one row: h (bf16-valued, length K), full-head and screen data.  surv (capacity cap_surv)
 * receives survivors in ascending order, sval their r16 rescored logits.  seeds: lower-bound
 * seed rows (may be NULL). */
void g4o_head_row(const float* h, int V, int K, const uint8_t* Wq, const uint16_t* Sq,
                  const float* coef, const uint8_t* data, const uint8_t cb8[8],
                  const int64_t* exc_ptr, const uint16_t* exc_col, const float* exc_delta,
                  const int* seeds, int nseeds, int limit, int* surv, float* sval, int cap_surv,
                  g4o_head_info* info);

/* ---- split-KV attention (engine/gemma4_engine.cpp:738-877, 1019-1059) ---- */
void g4o_attn_splitkv(const uint16_t* Kc, const uint16_t* Vc, int hd, int nh, int M,
                      const float* q, int ldq, const int* pos, const int* lo, const int* skip_lo,
                      const int* skip_hi, int kmin, int kmax, int T, float* out, int ldo,
                      float* part_m, float* part_l);

/* ---- prefill attention: attn_tile (E:1063-1083) and run_mh (E:1338-1349), row by row;
 * rows [M] at pos[m] attend [lo[m], pos[m]] ---- */
void g4o_attn_tile(const uint16_t* Kc, const uint16_t* Vc, int hd, int nh, int M, const float* q, int ldq,
                   const int* pos, const int* lo, float* out, int ldo);
/* skip_lo / skip_hi (optional): row m ignores positions skip_lo[m] .. skip_hi[m] (the sibling row) */
void g4o_attn_mh(const uint16_t* Kc, const uint16_t* Vc, int hd, int nh, int M, const float* q, int ldq,
                 const int* pos, const int* lo, const int* skip_lo, const int* skip_hi, float* out, int ldo);

/* ---- the Gemma-4-E2B layer layout (g4_oracle_gemma.c): 35 layers, head_dim 256 / 512,
 * KV sharing past layer 14, per-layer MLP widths, per-layer inputs (E:1222-1232, 1256-1405).
 * Tensors by pointer, as the checkpoint holds them: int4 [N][K/2] + bf16 scales [N][K/32],
 * bf16 vectors.  The per-layer embedding table is the rows ple_rows [nple][35 * 256] of the
 * ascending ids ple_ids (other rows zero). ---- */
typedef struct {
  const uint8_t* w;
  const uint16_t* s;
  int32_t N, K;
} g4o_q4;
typedef struct {
  g4o_q4 q, k, v, o, gate, up, down, pg, pp; /* k, v: layers 0..14 */
  const uint16_t *in_ln, *post_attn, *pre_ff, *post_ff, *post_ple, *qn, *kn;
  uint16_t scalar;
} g4o_glayer_in;
typedef struct {
  g4o_glayer_in L[35];
  g4o_q4 plproj;
  const uint16_t *plnorm, *fnorm, *E;
  int32_t V, nple;
  const int32_t* ple_ids;
  const uint16_t* ple_rows;
} g4o_gemma_in;
typedef struct g4o_gemma g4o_gemma;
g4o_gemma* g4o_gemma_new(const g4o_gemma_in* in, int ctx);
void g4o_gemma_free(g4o_gemma* g);
/* fwd of M <= 32 rows at pos0.. (T attention splits, sibling row index or -1); hbuf [M][1536]
 * receives the final-normed rows m >= hf (may be NULL) */
void g4o_gemma_forward(g4o_gemma* g, const int* toks, int M, int pos0, int T, int sibling, float* hbuf, int hf);
/* ENGINE_PREFILL_INT8=1 for the passes that follow: blocks of M >= 2 rows take W4A8 products */
void g4o_gemma_set_i8(g4o_gemma* g, int on);
/* the drafter's view of the layout: embedding, owner caches 13 / 14, RoPE tables, head dims */
void g4o_gemma_target(const g4o_gemma* g, const uint16_t** E, const uint16_t** K, const uint16_t** V,
                      const float** cs, const float** sn, int* hd);
/* E:1651: KV rows of slot `from` copied to slot `to` in the 15 owner caches */
void g4o_gemma_kv_move(g4o_gemma* g, int from, int to);
/* owner layer l's key (v = 0) or value (v = 1) cache [ctx][hd] */
const uint16_t* g4o_gemma_cache(const g4o_gemma* g, int l, int v);

/* ---- synthetic decoder stack + verify step (engine/gemma4_engine.cpp:1256-1502, 1617-1661) ---- */
typedef struct g4o_model g4o_model;
g4o_model* g4o_model_new(uint64_t seed, int V, int NL, int I, int ctx);
void g4o_model_free(g4o_model* m);
void g4o_model_fake_ctx(g4o_model* m, int n, uint64_t seed);
int g4o_model_bytes(const g4o_model* m, const char* what, void* dst, int64_t cap);
const void* g4o_model_ptr(const g4o_model* m, const char* what);

typedef struct {
  int nacc;      /* accepted drafts */
  int branch;    /* 0: chain a (or none), 1: branch b */
  int ncommit;   /* nacc + 1 */
  int commit[8]; /* committed tokens G[path] */
  int G[8];      /* greedy token per row, -1 where not evaluated */
  int fallback[8];
  int nsurv[8];
} g4o_verify_out;

/* one verify pass: toks[0] = confirmed token, toks[1..na] chain a, toks[na+1..na+nb] branch b;
 * rows are at positions pos0.. ; fills out and commits (KV compaction for branch b). */
void g4o_verify(g4o_model* m, const int* toks, int na, int nb, int pos0, int T,
                g4o_verify_out* out, float* hidden_out);
void g4o_verify_ex(g4o_model* m, const int* toks, int na, int nb, int pos0, int T, int allow_b,
                   g4o_verify_out* out, float* hidden_out);
/* the same with i8 = G_I8_ACTIVE in the decode: W4A8 linear layers for passes of M >= 2 rows */
void g4o_verify_i8(g4o_model* m, const int* toks, int na, int nb, int pos0, int T, int allow_b, int i8,
                   g4o_verify_out* out, float* hidden_out);

/* prefill (E:1594-1599, ENGINE_PREFILL_INT8=1): toks[0..n) at pos0.. in blocks of pfb rows;
 * fills the KV cache; hlast (optional) receives the final-normed hidden row of the last token */
void g4o_prefill(g4o_model* m, const int* toks, int n, int pos0, int pfb, int T, float* hlast);
void g4o_prefill_ex(g4o_model* m, const int* toks, int n, int pos0, int pfb, int T, int i8, float* hlast);

/* the head of one final-normed row (E:1406-1500); toks[0..nt) (nt <= 8) seed the screen */
int g4o_model_head(g4o_model* m, const float* h, const int* toks, int nt);

/* forward of M rows that fills the KV cache only (want = false) */
void g4o_forward_fill(g4o_model* m, const int* toks, int M, int pos0, int T);

/* ---- MTP drafter step (E:1534-1563) on the synthetic target; see g4_oracle_draft.c ---- */
typedef struct g4o_drafter g4o_drafter;
g4o_drafter* g4o_drafter_new(uint64_t seed, int V);
/* a drafter checkpoint (E:1519-1528), tensors as stored (bf16; token ordering int64) */
typedef struct {
  const uint16_t *pre, *post, *cent, *emb, *dnorm;
  const int64_t* order;
  const uint16_t *q[4], *o[4], *gate[4], *up[4], *down[4];
  const uint16_t* nv[4][5]; /* input, post-attention, pre-FFN, post-FFN layernorms; q_norm */
  uint16_t scalar[4];
  int32_t V, C, hd[4];
} g4o_drafter_in;
g4o_drafter* g4o_drafter_load(const g4o_drafter_in* in);
void g4o_drafter_free(g4o_drafter* d);
const void* g4o_drafter_ptr(const g4o_drafter* d, const char* what);
int g4o_model_ctx(const g4o_model* m);
/* b16_rows (E:586-614): y [N] = W [N][K] bf16 . x [K] */
void g4o_b16_gemv(const uint16_t* W, int N, int K, const float* x, float* y);
/* one draft step: returns the draft token; b_out [1536], sec, gap as E:1553, 1559 */
int g4o_gemma_draft_step(const g4o_gemma* g, const g4o_drafter* d, int tok, const float* h, int pos, int P, int T,
                         float* b_out, int* sec_out, float* gap_out);
int g4o_draft_step(const g4o_model* m, const g4o_drafter* d, int tok, const float* h, int pos, int P, int T,
                   float* b_out, int* sec, float* gap);

/* ---- seeded input generators (g4_rng.h formulas) ---- */
uint64_t g4o_stream(uint64_t seed, uint64_t tag);
void g4o_gen_normal_f32(uint64_t seed, int64_t n, float scale, float* out);
void g4o_gen_normal_bf16(uint64_t seed, int64_t n, float scale, uint16_t* out);
void g4o_gen_bytes(uint64_t seed, int64_t n, uint8_t* out);
void g4o_gen_scales(uint64_t seed, int64_t n, float lo, float span, uint16_t* out);
void g4o_gen_ints(uint64_t seed, int64_t n, int32_t lo, int32_t hi, int32_t* out);

#ifdef __cplusplus
}
#endif
#endif
