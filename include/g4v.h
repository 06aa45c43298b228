/* g4v.h -- C ABI of the MI355X (gfx950) speculative-verify path.
 *
 * Drop-in boundary for the verify hot path of dayaswaroopchavali/gemma4-e2b-laptop-cpu.
 * Every entry point replaces a kernel-call surface of the reference engine (citations
 * are reference file:line, E = engine/gemma4_engine.cpp).  Plain pointers and sizes only;
 * the library owns all device memory.  Host pointers are used for small inputs/outputs;
 * results are bit-identical to the reference's exact-float path (ENGINE_DECODE_INT8=0) and,
 * with g4v_set_prefill_int8 / g4v_set_decode_int8, to its W4A8 prefill and decode (E:1210, 1600).
 *
 * Errors: every function returns 0 on success, a negative G4V_E* code otherwise, and never
 * exits the process; g4v_error() describes the last failure of a context.
 * Threading: one host thread per context; calls are stream-ordered and synchronous on return.
 */
#ifndef G4V_H
#define G4V_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define G4V_OK 0
#define G4V_E_ARG (-1)      /* invalid argument or shape */
#define G4V_E_HIP (-2)      /* HIP runtime failure */
#define G4V_E_STATE (-3)    /* call out of order (e.g. no model) */
#define G4V_E_NOMEM (-4)    /* device allocation failed */

typedef struct g4v_ctx g4v_ctx;

/* Context on HIP device `device` (the GPU replaces the reference's Pool, E:73-141). */
int g4v_create(int device, g4v_ctx** out);
void g4v_destroy(g4v_ctx* c);
const char* g4v_error(const g4v_ctx* c);
/* device name, compute units, max dynamic LDS bytes per block */
int g4v_device_info(g4v_ctx* c, char* name, int cap, int* cus, int* lds_per_block);

/* ---- int4 G32 matrices: Q4 handle (E:174-175), w4::gemm_rows_tile (engine/w4g32_avx2.h:64-96)
 * through lin1/lin_multi (E:310-317).  w: [N][K/2] bytes, low nibble = even k, value q+8;
 * s: [N][K/32] bf16 scales.  Returns a handle >= 0. K % 256 == 0. */
int g4v_w4_upload(g4v_ctx* c, const uint8_t* w, const uint16_t* s, int N, int K);
/* y[m][n] for M <= 8 rows of x [M][K] (fp32), bit-identical to gemm_rows_tile */
int g4v_w4g32_gemm(g4v_ctx* c, int h, const float* x, int M, float* y);
/* lin_multi (E:310-317): 1 to 3 matrices with the same K over the same rows in one launch (the
 * q / k / v phase); y[j] [M][N_j] for handle h[j] */
int g4v_w4g32_gemm_multi(g4v_ctx* c, int nmat, const int* h, const float* x, int M, float* const* y);
/* same GEMV with x and y already on the device; times `iters` launches, returns us/launch */
int g4v_w4g32_bench(g4v_ctx* c, int h, int M, int iters, float* us_per_launch);
/* the residual and RMS-norm block between two sub-blocks fused into the next product, as the
 * verify pass runs it: mode 1 (after attention, E:1358-1361):
 *   x1 = r16(xin + r16(rms(r16(o), w1))), y = W r16(rms(x1, w2));
 * mode 2 (after the MLP, E:1375-1378 and E:1390-1404 with the per-layer-embedding branch zero):
 *   x1 = r16(r16(xin + r16(rms(r16(o), w1))) * scalar), y = W rms(x1, w2);
 * rms(v, w) = (v * r) * w with r = 1 / sqrtf((float)(sum of squares / 1536) + 1e-6f), the sum
 * in double over 16 lanes (E:326-352).  o, xin, x1: [M][1536]; w1, w2: [1536]; the handle's
 * K = 1536, N % 64 == 0; 1 <= M <= 8.  rows_per_block (1..4) and tile_rows (32, 64) choose the
 * launch shape the verify pass tunes per product. */
int g4v_w4g32_norm_gemm(g4v_ctx* c, int h, int mode, const float* o, const float* xin, const float* w1,
                        const float* w2, float scalar, int M, int rows_per_block, int tile_rows, float* y, float* x1);

/* ---- W4A8: w4a8::quant (engine/w4a8_avx2.h:30-42) and w4a8::tile<MT> over all rows as
 * i8_task runs it (engine/w4a8_avx2.h:46-61, E:303-309), on a handle of g4v_w4_upload with
 * N % 16 == 0.  The engine takes this path for prefill and, with ENGINE_DECODE_INT8 set, for
 * M >= 2 decode rows (E:311).  1 <= M <= 8192.
 * quant: q [M][K] int8, sx [M][K/32] (amax / 127), sum [M][K/32] (sum of the integers). */
int g4v_w4a8_quant(g4v_ctx* c, const float* x, int M, int K, int8_t* q, float* sx, int32_t* sum);
/* y[m][n] (fp32, [M][N]) bit-identical to quant + tile */
int g4v_w4a8_gemm(g4v_ctx* c, int h, const float* x, int M, float* y);
/* quant + GEMM with the operands already on the device; times `iters` runs, us per run */
int g4v_w4a8_bench(g4v_ctx* c, int h, int M, int iters, float* us_per_launch);
/* ---- the components on their own, device-timed (the reference times its kernels alone in
 * bench/attn_bench.cpp:16-34, warm and cold): *us = the mean of `iters` launches, each between two
 * events on the library's stream.  cold = 0: the launches repeat on operands that stay in the
 * caches; cold = 1: a read of 512 MB (twice the last-level cache) before each launch, outside the
 * events, evicts them.
 * g4v_w4g32_time: one launch of the verify pass's row-tile GEMV over nmat matrices of the same K
 * (N % 64 == 0; two of them = the fused gate/up pair) on M staged rows (E:1289, 1363-1371); flags
 * bit 0 = cold, bit 1 = the W4A8 product instead (lin_multi with G_I8_ACTIVE, E:311; the rows
 * quantised in the product's blocks). */
int g4v_w4g32_time(g4v_ctx* c, int nmat, const int* h, int M, int iters, int flags, float* us);
/* split-KV attention (k_attn_split + k_attn_merge) of M rows at positions npos - M .. npos - 1 over
 * keys [0 or pos - 511 with window, pos], nsplit splits, on a device cache of npos positions
 * (E:1305-1327, the ATT_PAR path) */
int g4v_attn_time(g4v_ctx* c, int npos, int M, int nsplit, int window, int iters, int cold, float* us);
/* the head (screen, threshold, survivors, rescore, and the full head on an overflow) of one row h
 * [1536] (E:1406-1500); nsurv / fallback as g4v_head_argmax reports them for that row */
int g4v_head_time(g4v_ctx* c, const float* h, int iters, int cold, float* us, int* nsurv, int* fallback);

/* ---- split-KV attention: attn_task + attn_merge (E:743-877, E:1019-1059) with the
 * reference's split geometry [kmin + t*len/T, kmin + (t+1)*len/T).  Kc, Vc: [npos][hd] bf16;
 * q: [M][nh*hd] fp32; per row: pos, lo, skip_lo, skip_hi (attn_allowed, E:740).
 * out: [M][nh*hd] fp32, rounded to bf16 values.  hd 256 or 512 (the global layers of the
 * Gemma-4-E2B layout, E:1225), nh == 8, M <= 8, nsplit <= 16. */
int g4v_attn_splitkv(g4v_ctx* c, const uint16_t* Kc, const uint16_t* Vc, int npos, int hd, int nh, int M,
                     const float* q, const int* pos, const int* lo, const int* skip_lo, const int* skip_hi,
                     int kmin, int kmax, int nsplit, float* out);
/* The same attention on device buffers, allocating nothing (no hipMalloc, hipFree or allocating
 * library call): Kc, Vc, q and out are device pointers (same layouts as above), pos / lo /
 * skip_lo / skip_hi host arrays.  No counterpart in the reference: it is for callers that cannot
 * allocate (tight serving loops, harnesses that forbid allocation).  The call is synchronous: it
 * launches on the context's own stream and waits for it, so it is not for a caller's stream
 * capture.  Its scratch (the relaid key / value rows and the split partials, 5.3 MB) is a
 * file-scope device array, one per GPU, held until the process ends and shared by every call on
 * that GPU: npos <= 4096; calls that overlap on one GPU race. */
int g4v_attn_splitkv_noalloc(g4v_ctx* c, const uint16_t* Kc, const uint16_t* Vc, int npos, int hd, int nh, int M,
                             const float* q, const int* pos, const int* lo, const int* skip_lo, const int* skip_hi,
                             int kmin, int kmax, int nsplit, float* out);

/* ---- certified head (E:1232-1244 build; E:1406-1500 head_group).  E: [V][1536] bf16 output
 * matrix; builds the int4 screen, the exp3 codebook + exception list and the cap table. */
int g4v_head_build(g4v_ctx* c, const uint16_t* E, int V);
/* head of M <= 4 final-normed rows h [M][1536] (bf16 values): greedy token G[m] (lowest-index
 * tie rule), survivor count, 1 when the full head was evaluated. */
int g4v_head_argmax(g4v_ctx* c, const float* h, int M, int* G, int* nsurv, int* fallback);
/* survivors of row m of the last g4v_head_argmax (ascending index) and their r16 logits */
int g4v_head_survivors(g4v_ctx* c, int m, int* idx, float* val, int cap, int* n);

/* ---- synthetic decoder stack (35-layer Gemma-4-E2B-shaped, int4 G32, hd 256, 8q/1kv heads,
 * l % 5 != 4 sliding-window 512) generated on device from `seed`. */
int g4v_model_synth(g4v_ctx* c, uint64_t seed, int V, int NL, int I, int ctxcap);
/* The same stack from the caller's own weights (the checkpoint the engine maps, E:166-176).
 * g4v_model_create allocates an empty stack and zeroes the KV cache. Then set the
 * embedding / tied output matrix E [V][1536] bf16 (E:1262-1267, E:1406; this also builds the
 * certified head), the 7 matrices of every layer in the Q4 byte layout (j: 0 q [2048x1536],
 * 1 k [256x1536], 2 v [256x1536], 3 o [1536x2048], 4 gate [Ix1536], 5 up [Ix1536],
 * 6 down [1536xI]; E:1289, 1356, 1366, 1373), the six norm vectors of every layer (in_ln,
 * post_attn, pre_ff, post_ff [1536]; q_norm, k_norm [256]) with the layer scalar and its
 * attention type (sliding window 512 or global), and the final norm.  g4v_verify_step
 * refuses a stack with any matrix or the embedding unset. */
int g4v_model_create(g4v_ctx* c, int V, int NL, int I, int ctxcap);
int g4v_model_set_embed(g4v_ctx* c, const uint16_t* E);
int g4v_model_set_matrix(g4v_ctx* c, int layer, int j, const uint8_t* w, const uint16_t* s);
int g4v_model_set_norms(g4v_ctx* c, int layer, const float* const nv[6], float scalar, int sliding);
int g4v_model_set_final_norm(g4v_ctx* c, const float* w);
/* ---- the Gemma-4-E2B layer layout (E:1222-1232, fwd E:1256-1405): 35 layers, head_dim 256
 * (l % 5 != 4, window 512) or 512 (global; RoPE theta 1e6 on the first quarter of the
 * frequencies), k / v projections and caches in layers 0..14 only (later layers read layer 13's
 * or 14's cache), the MLP width mlp[l] of each layer, and the per-layer-input branch.  After
 * this call: g4v_model_set_embed, g4v_model_set_final_norm, g4v_model_set_matrix for j = 0 q,
 * 1 k, 2 v (layers < 15), 3 o, 4 gate, 5 up, 6 down, 7 per_layer_input_gate [256][1536],
 * 8 per_layer_projection [1536][256], g4v_model_set_norms_gemma, g4v_model_set_ple and the
 * table rows; then g4v_prefill, g4v_verify_step (a chain of up to 7 drafts) and
 * g4v_verify_sibling run that layout. */
int g4v_model_create_gemma(g4v_ctx* c, int V, const int* mlp, int ctxcap);
/* the same layout with every tensor generated on the device from seed (no reference
 * counterpart: the benchmark's Gemma-4-E2B workload without a checkpoint) */
int g4v_model_synth_gemma(g4v_ctx* c, uint64_t seed, int V, const int* mlp, int ctxcap);
/* nv: in_ln, post_attn, pre_ff, post_ff, post_per_layer_input_norm [1536 each], q_norm, k_norm
 * [hd each; k_norm null past layer 14]; scalar: layer_scalar */
int g4v_model_set_norms_gemma(g4v_ctx* c, int layer, const float* const nv[7], float scalar);
/* per_layer_model_projection (int4 [8960][1536], scales [8960][48]) and per_layer_projection_norm [256] */
int g4v_model_set_ple(g4v_ctx* c, const uint8_t* w, const uint16_t* s, const float* plnorm);
/* rows tok0 .. tok0 + n - 1 of the per-layer embedding table, bf16 [n][35 * 256] (zero until set) */
int g4v_model_set_ple_rows(g4v_ctx* c, int tok0, int n, const uint16_t* rows);
/* KV rows [pos0, pos0 + n) of one layer, bf16 [n][256] each: a cache filled elsewhere
 * (the engine's prefill, E:1328-1336) */
int g4v_model_set_kv(g4v_ctx* c, int layer, int pos0, int n, const uint16_t* K, const uint16_t* V);
/* E:1249-1250 ENGINE_FAKE_CTX: first n KV positions of every layer from the LCG seeded `seed`
 * (the reference's seed is 12345); on the Gemma-4-E2B layout the 15 owner caches (layers 0..14,
 * each at its head dim), which are the caches main() fills */
int g4v_model_fake_ctx(g4v_ctx* c, int n, uint64_t seed);
/* copy a named model array to the host ("E", "W<l>_<j>", "S<l>_<j>", "N<l>_<t>", "KC", "VC", "fnorm",
 * the Gemma layout's owner caches "GK<l>" / "GV<l>" [ctxcap][hd] (l < 15),
 * the head screen "Wq" [V][768], "Sq" [V][48] bf16, "coef" [V] f32, in the reference's layouts,
 * and the exact head's device forms: "cb" the 8-entry exponent codebook, "dec" the decoded bf16
 * weights [V][24][8][8] in the fma-lane order, "x3sm" [V][24][8] uint2 and "x3ix" [V][24][8]
 * uint32 the exp3 form the full head streams) */
int g4v_model_read(g4v_ctx* c, const char* what, void* dst, size_t cap, size_t* nbytes);

/* ---- one verify pass (fwd E:1256-1502 + lazy head E:1453-1488 + accept E:1647-1661).
 * toks[0] confirmed token, toks[1..na] chain a, toks[na+1..na+nb] branch b: a chain of up to 7
 * drafts (nb = 0, E:1514), or two branches of up to 4 drafts each (na + nb <= 7);
 * rows sit at positions pos0.. ; nsplit = attention splits (the reference's thread count). */
typedef struct {
  int nacc;      /* accepted drafts */
  int branch;    /* 0: chain a, 1: branch b */
  int ncommit;   /* nacc + 1 tokens committed */
  int commit[8];
  int G[8];      /* greedy token per row, -1 where not evaluated */
  int fallback[8];
  int nsurv[8];
} g4v_verify_result;
int g4v_verify_step(g4v_ctx* c, const int* toks, int na, int nb, int pos0, int nsplit, g4v_verify_result* out,
                    float* hidden);
/* the engine's pass with a sibling row (E:1634-1655): toks[0] confirmed, toks[1..nd] MTP drafts
 * (nd 1 or 2), toks[nd+1] the drafter's runner-up for the first draft, at RoPE position pos0 + 1
 * and slot pos0 + nd + 1, attending rows up to pos0 and itself (E:1345).  allow_hit is the
 * engine's (TREE || (P + 1 + sibling <= ATT_PAR && gap1 >= 0.25)) of E:1650: when set and row 0's
 * token equals the sibling's (but not the first draft's), the sibling commits (branch 1, its KV
 * moved to slot pos0 + 1); otherwise only chain acceptance applies.  Replaces fwd(block, nd + 2,
 * P + 1, true, 0, nullptr, sibling) and the tree-hit test of engine/gemma4_engine.cpp:1647-1656. */
int g4v_verify_sibling(g4v_ctx* c, const int* toks, int nd, int pos0, int nsplit, int allow_hit,
                       g4v_verify_result* out, float* hidden);
/* Verify steps run as one captured HIP graph per shape (rows, branches, splits) from the
 * second call of that shape on (the engine's persistent pool + job word, E:73-141, becomes a
 * graph launch).  on = 0 launches every kernel from the host instead. */
int g4v_set_graphs(g4v_ctx* c, int on);
/* E:1210 G_I8 (ENGINE_PREFILL_INT8=1, the default here): g4v_prefill multiplies blocks of two
 * rows or more W4A8 (lin_multi, E:311); 0: exact float throughout, the reference's default */
int g4v_set_prefill_int8(g4v_ctx* c, int on);
/* E:1600 DEC_I8 (ENGINE_DECODE_INT8, on by default in the reference when ENGINE_PREFILL_INT8=1):
 * on = 1 with prefill int8 on keeps G_I8_ACTIVE in the decode, so verify passes of two rows or
 * more (g4v_verify_step / g4v_verify_sibling) multiply W4A8 as lin_multi does (E:311), on both the
 * Gemma layout and the synthetic stack (the same passes with W4A8 products; the values equal the
 * engine's unfused structure of that mode, E:1268-1289, 1363-1388).  Off by default here (exact
 * float decode). */
int g4v_set_decode_int8(g4v_ctx* c, int on);
/* E:1516 SAMEPOS (ENGINE_DRAFT_SAMEPOS=1): g4v_draft_mtp runs every step of a chain at query
 * position P + 1 (its RoPE angle and sliding window), as draft_step(..., SAMEPOS ? P + 1 :
 * P + 1 + j, ...) does (E:1633); 0 (the default): step j at P + 1 + j. */
int g4v_set_draft_samepos(g4v_ctx* c, int on);

/* ---- prefill: run_req's prompt loop (E:1594-1599) with ENGINE_PREFILL_INT8=1, i.e. fwd
 * (E:1256-1405) over blocks of pfb rows (ENGINE_PREFILL_BLOCK, 32 by default), W4A8 linear layers
 * (w4a8::quant + tile, engine/w4a8_avx2.h:30-61) for blocks of M >= 2 rows, and the engine's
 * attention path per block: attn_tile (E:1063-1083), run_mh (E:1338-1349) or split-KV with
 * nsplit splits (E:1305-1327).  toks[0..n) sit at positions pos0..; every layer's KV rows are
 * written.  G0 = greedy token of the last row (the first generated token, E:1601), hidden
 * (optional, [1536]) = that row's final-normed state.  Needs a model (g4v_model_synth or
 * g4v_model_create + set calls) and pos0 + n <= ctxcap. */
int g4v_prefill(g4v_ctx* c, const int* toks, int n, int pos0, int pfb, int nsplit, int* G0, float* hidden);

/* ---- MTP drafter: draft_step (E:1534-1563) chained as run_req chains it (E:1631-1646), on the
 * device.  g4v_drafter_synth builds a synthetic drafter for the current model (4 layers of
 * hidden 256, 4 query heads of head_dim 256 attending the target's KV cache of layers 13 and
 * 14, FFN 2048, V / 128 centroids, bf16 weights from `seed`); it needs V = 128 C with
 * 32 <= C <= 4096, C % 16 == 0, and at least 15 target layers.
 * g4v_draft_mtp runs k steps: step j drafts from token t_j (t_0 = tok) and hidden state h_j
 * (h_0 = h, or the last g4v_verify_step's committed hidden state when h is null; h_j = the
 * previous step's output) at query position P + 1 + j over the target keys [lo, P] with nsplit
 * splits (the reference's pool size, 6 by default).  drafts[j] = t_{j+1}; sec[j] / gap[j]
 * (optional) = runner-up token and score gap (g_sec, g_gap); hidden (optional, [1536]) = the
 * last step's output state.  1 <= k <= 8. */
int g4v_drafter_synth(g4v_ctx* c, uint64_t seed);
/* A drafter checkpoint (replaces E:1519-1528, the ENGINE_DRAFTER_DIR / ENGINE_DRAFTER_INDEX
 * loader of main()): bf16 tensors as stored.  pre_projection [256][3072], post_projection
 * [1536][256], masked_embedding.centroids [C][256], model.embed_tokens [V][256], model.norm [256],
 * masked_embedding.token_ordering int64 [V]; per layer l: q_proj [4 hd][256], o_proj [256][4 hd],
 * gate_proj / up_proj [2048][256], down_proj [256][2048], norms nv[l] = input_layernorm,
 * post_attention_layernorm, pre_feedforward_layernorm, post_feedforward_layernorm [256] and
 * q_norm [hd], layer_scalar.  hd[l] = 256 for l < 3; layer 3 has the head dim of the target's
 * layer 14 (512 on the Gemma-4-E2B layout, 256 on the synthetic stack).  V = 128 C. */
typedef struct {
  const uint16_t *pre, *post, *cent, *emb, *norm;
  const int64_t* order;
  const uint16_t *q[4], *o[4], *gate[4], *up[4], *down[4];
  const uint16_t* nv[4][5];
  uint16_t scalar[4];
  int32_t C, hd[4];
} g4v_drafter_tensors;
int g4v_drafter_load(g4v_ctx* c, const g4v_drafter_tensors* t);
int g4v_draft_mtp(g4v_ctx* c, int tok, const float* h, int P, int k, int nsplit, int* drafts, int* sec, float* gap,
                  float* hidden);

/* ---- prefix cache (run_req, E:1568-1593, E:1671): the active KV cache plus nslot - 1 stored
 * conversations (ENGINE_SLOTS; each a full cache copy on the device), reuse threshold min_reuse
 * (ENGINE_SLOT_MIN_REUSE, 32).  Per request: g4v_slot_begin picks the conversation that shares
 * the longest prefix with toks (switching slots, or parking the active one in the least recently
 * used slot when nothing reaches min_reuse) and returns start = the positions whose KV is reused
 * (at most n - 1) and the slot used (0 = the active one); the caller prefills toks[start..n) at
 * position start and decodes; g4v_slot_end records what the cache now holds: the prompt and
 * gen[i] for i <= P - n, valid up to position P. */
int g4v_slots_init(g4v_ctx* c, int nslot, int min_reuse);
int g4v_slot_begin(g4v_ctx* c, const int* toks, int n, int* start, int* slot_used);
int g4v_slot_end(g4v_ctx* c, const int* toks, int n, const int* gen, int ngen, int P);

/* ---- prompt-lookup drafter (run_req, E:1624-1628) over a history kept on the device.
 * history_set: seq = toks[0..L), the prompt followed by the generated tokens (E:1625). */
int g4v_history_set(g4v_ctx* c, const int* toks, int L);
/* Appends append[0..na) (the round's committed tokens, E:1659; na <= 16) to seq, then drafts
 * as the reference does with NG_N = n and NG_LEN = maxlen (E:1514): the tokens that followed the
 * most recent earlier occurrence of seq's last n tokens, at most maxlen of them and none past
 * the end of seq.  *nd = 0 when n <= 0, |seq| <= n or the n-gram has no earlier occurrence.
 * n <= 256, maxlen <= 16 (the reference caps NG_LEN at 7). */
int g4v_prompt_lookup(g4v_ctx* c, const int* append, int na, int n, int maxlen, int* drafts, int* nd);
/* *L = |seq|; copies min(cap, |seq|) tokens of it to toks (may be null) */
int g4v_history_read(g4v_ctx* c, int* toks, int cap, int* L);

/* ---- measurement (replaces the reference's PROF_NM / T_* stage timers, E:66-70, E:1085):
 * per-kernel-class HIP events on the library's stream.  Classes: 0 gemv_qkv, 1 gemv_o,
 * 2 gemv_gateup, 3 gemv_down, 4 attn, 5 rows (norm/rope/embed), 6 head_screen, 7 head_select,
 * 8 head_rescore, 9 head_full, 10 head_tie, 11 accept, 12 head_pass2.  Bit t of `mask` enables
 * class t; the totals (ms, algorithmic bytes, launches) reset on every g4v_profile call. */
#define G4V_PROF_NTAGS 13
int g4v_profile(g4v_ctx* c, unsigned mask);
int g4v_profile_read(g4v_ctx* c, double* ms, double* bytes, long long* count, int n);
/* the last g4v_prefill's head row (its G0): screen survivors and whether it fell back to the full
 * head (more than 30,000 survivors), as g4v_verify_result reports them per row -- what the
 * reference's SCREEN statistics count per evaluated row (E:1472 scr_rows / scr_surv / scr_max,
 * E:1489 scr_fallback, printed at E:1690) */
int g4v_prefill_head_stats(g4v_ctx* c, int* nsurv, int* fallback);

/* device read (mode 0) or copy (mode 1, read + write bytes counted) bandwidth in GB/s over a
 * buffer of `bytes` (>= 1 MiB, a multiple of 16) streamed `passes` times.  No counterpart in the
 * verify path: the device restatement of the reference's host probe bench/stream_bw.cpp:10-19
 * (the bandwidth figures beside the roofline), and the copy of known bytes that calibrates the
 * FETCH_SIZE / WRITE_SIZE counters. */
int g4v_hbm_stream(g4v_ctx* c, size_t bytes, int passes, int mode, double* gbps);

/* wait for all work of the context */
int g4v_sync(g4v_ctx* c);

/* host-side self check of the expf restatement used by the split merge: mismatches against
 * the linked libm expf over float bit patterns [lo, hi] (step `stride`) */
long long g4v_expf_selftest(uint32_t lo, uint32_t hi, uint32_t stride);

#ifdef __cplusplus
}
#endif
#endif
