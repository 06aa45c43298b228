// g4v_layer.h -- per-step parameters and the layer / attention / acceptance kernels.
#pragma once
#include "g4v_internal.h"

namespace g4v {

// Rows of one verify pass (written by the host before every step).  Row 0 is the
// confirmed token, rows 1..na chain a, rows na+1..na+nb branch b.  Cache slot of row r is
// pos0 + r; its RoPE position is rope[r]; attention skips [skip_lo, skip_hi] (E:1326).
struct StepDev {
  int M, na, nb, pos0;
  int toks[MAXM];
  int rope[MAXM];
  int skip_lo[MAXM];
  int skip_hi[MAXM];
  int b_ok;  // 0: branch b is never committed (the sibling row when the tree hit is not taken)
};

struct VerifyResultDev {
  int nacc, branch, ncommit, pad;
  int commit[MAXM];
  int G[MAXM];
  int fallback[MAXM];
  int nsurv[MAXM];
  int hrows[MAXM];  // rows evaluated by the second head pass
  int hcount;       // how many
  int pad2[3];
};

// E:326-343 ss_avx2: lane t (0..15) accumulates x[16 s + t]^2 in double over steps s;
// s[k][l] = lane 4k + l; a[l] = (s[0][l]+s[1][l])+(s[2][l]+s[3][l]); ss = (a0+a2)+(a1+a3).
// x is in LDS; red16 is LDS scratch; every thread returns ss.
__device__ inline double block_sumsq(const float* x, int n, double* red16) {
  if (threadIdx.x < 16) {
    double s = 0;
#pragma unroll 16
    for (int i = threadIdx.x; i < n; i += 16) {  // loads run ahead; the FMA chain stays in order
      const double d = (double)x[i];
      s = fma(d, d, s);
    }
    red16[threadIdx.x] = s;
  }
  __syncthreads();
  double a[4];
  for (int l = 0; l < 4; ++l) a[l] = (red16[l] + red16[4 + l]) + (red16[8 + l] + red16[12 + l]);
  const double ss = (a[0] + a[2]) + (a[1] + a[3]);
  __syncthreads();
  return ss;
}

// E:345: r = 1 / sqrtf((float)(ss / n) + 1e-6)
__device__ __forceinline__ float rms_inv(double ss, int n) { return 1.0f / sqrtf((float)(ss / n) + 1e-6f); }

constexpr int ROW_THREADS = 256;

// per-layer pointers for the layer kernels
struct LayerNorms {
  const float* in_ln;      // [H]
  const float* post_attn;  // [H]
  const float* pre_ff;     // [H]
  const float* post_ff;    // [H]
  const float* qn;         // [HD]
  const float* kn;         // [HD]
  const float* qnp;        // qn, kn in the 16-lane head order (head16_index)
  const float* knp;
  float scalar;
  int sliding;
};

// xa / att / act below are written in the staged GEMV input layout (staged_index) with their
// group sums (xgs, attgs)
// rope: [2 layer types][cos, sin][ctxcap][HD/2]; ropestep: [2][MAXM][cos | sin][HD/2] of the step's rows
void launch_embed(const uint16_t* E, const StepDev* sp, const float* in_ln, float sqh, float* x, float* xa, float* xgs,
                  const float* rope, int ctxcap, float* ropestep, int M, hipStream_t st);
// verify-pass attention on the raw projections q, k, v: q/k norm, RoPE and the cache rows of
// the pass (E:1307-1324) fused into the split kernel; the split partials po / pm / pl are
// merged by their consumer, the o projection (GemvTArgs::mrg_po)
void launch_attn(uint16_t* KC, uint16_t* VC, const float* q, const float* k, const float* v, const LayerNorms& ln,
                 const float* ropestep, const StepDev* sp, int sliding, int T, float* po, float* pm, float* pl, int M,
                 hipStream_t st);
void launch_post_attn(const float* o, float* x, float* xa, float* xgs, const LayerNorms& ln, int M, hipStream_t st);
void launch_post_ff(const float* o, float* x, float* xa, float* xgs, const LayerNorms& ln, const float* next_in_ln,
                    const float* fnorm, float* h, float* hn, int M, hipStream_t st);
void launch_branch(const StepDev* sp, const int* best1, const float* h, const float* hn, float* h2, float* hn2,
                   VerifyResultDev* res, hipStream_t st);
void launch_accept(const StepDev* sp, const int* best1, const int* best2, const int* cnt1, const int* cnt2,
                   VerifyResultDev* res, uint16_t* KC, uint16_t* VC, int NL, int kvcap, hipStream_t st);

// dst = the 256-vector src in the 16-lane head order (head16_index)
void launch_perm16(const float* src, float* dst, hipStream_t st);

// exchange the contents of two device buffers of `bytes` (a multiple of 16)
void launch_swap16(void* a, void* b, size_t bytes, hipStream_t st);

// synthetic weights (same formulas as the oracle's generator)
void launch_gen_bf16_normal(uint16_t* out, size_t n, uint64_t seed, float scale, hipStream_t st);
void launch_gen_w4(uint8_t* w, uint16_t* s, size_t nbytes, size_t nscales, uint64_t sw, uint64_t ss,
                   hipStream_t st);

// prefill (g4v_prefill.hip).  Rows r of a prompt of n rows sit at positions pos0 + r, in blocks
// of pfb rows; a kernel over a segment of rows [r0, r0 + M) takes its rows' paths from this.
// rows pos0 .. pos0 + n - 1 in blocks of pfb; sib >= 0: that row is the engine's sibling row
// (E:1292, 1340-1345): RoPE position and window from pos0 + 1, positions pos0 + 1 .. its own slot - 1
// skipped, and its pass never takes attn_tile (E:1328)
struct PfGeom {
  int n, pos0, pfb, sib;
};
void launch_pf_embed(const uint16_t* E, const int* toks, const float* in_ln, float sqh, float* x, float* a, int M,
                     hipStream_t st);
// q [M][8 hd] normed + rotated in place; k, v [M][hd] normed into the cache rows P0 .. (own = 0:
// q only, the layer reads another layer's cache); row sib (>= 0) is rotated at position P0 + 1
// (the sibling row).  hd 256 or 512; cs / sn the layer type's RoPE tables [ctx][hd / 2].
void launch_pf_qkv(float* q, const float* k, const float* v, const float* qn, const float* kn, const float* cs,
                   const float* sn, uint16_t* KC, uint16_t* VC, int P0, int M, hipStream_t st, int sib = -1,
                   int hd = HD, int own = 1, const int* dpos = nullptr);
// score scratch (floats) of M rows starting at position Pb
long long pf_score_floats(int M, int Pb, int sliding);
// attn_tile / run_mh attention of segment rows [r0, r0 + M): q [n][2048] (row r at r), att likewise
// staged: att rows in the staged GEMV input layout (staged_index) instead of plain.
// dpos (launch_pf_qkv too): not null, g.pos0 (P0) is read from that device word when the kernels
// run, so that a captured pass serves every position; the grid then covers positions below maxpos.
void launch_pf_attn(const float* q, const uint16_t* KC, const uint16_t* VC, float* S, float* att, const PfGeom& g,
                    int r0, int M, int sliding, hipStream_t st, bool staged = false, int hd = HD,
                    const int* dpos = nullptr, int maxpos = 0);
void launch_pf_post_attn(const float* o, float* x, float* a, const float* w1, const float* w2, int M, hipStream_t st);
void launch_pf_act(const float* g, const float* u, float* act, size_t n, hipStream_t st);
void launch_pf_post_ff(const float* o, float* x, float* a, const float* w1, const float* next_in_ln,
                       const float* fnorm, float scalar, float* h, int hrow, int M, hipStream_t st,
                       float* hn = nullptr);
// the per-layer-input branch of the Gemma-4-E2B layout: pli [M][35][256] from the projection rows
// pr [M][35 * 256] (E:615-660); g2 [M][256] for layer l from the gate rows pgv (E:405-443)
void launch_gm_ple(const float* pr, const int* toks, const uint16_t* ple, const float* plnorm, float* pli, int M,
                   hipStream_t st);
void launch_gm_pg_act(const float* pgv, const float* pli, int l, int M, float* g2, hipStream_t st);
// E:1651 for an owner cache of head dim hd (256 or 512): the committed branch rows moved into place
void launch_kv_compact_hd(const StepDev* sp, const VerifyResultDev* res, uint16_t* K, uint16_t* V, int hd,
                          hipStream_t st);

struct AttnGeom;

// MTP drafter (g4v_mtp.hip): one bf16 product y[n] = W[row(n)] . input, input prologue `pro`
// (0 x, 1 rms(x, nw), 2 r16(rms(x, nw)), 3 [r16(E[*tok] sqrt H), x], 4-6 the layer's residual
// blocks folded in front, see g4v_mtp.hip) and epilogue `epi` (0 store, 1 r16, 2 gate/up
// activation with W2 the up matrix)
struct B16Launch {
  const uint16_t* W = nullptr;
  const uint16_t* W2 = nullptr;
  const int* rows = nullptr;
  const int* top = nullptr;
  const int* order = nullptr;
  int N = 0, K = 0;
  const float* x = nullptr;
  const float* nw = nullptr;
  const uint16_t* E = nullptr;
  const int* tok = nullptr;
  float* y = nullptr;
  float* xout = nullptr;
  const float* yin = nullptr;
  const float* w1 = nullptr;
  float* dxout = nullptr;
  float scalar = 0.f;
  int pro = 0, epi = 0;
};
void launch_b16(const B16Launch& L, hipStream_t st);
// q heads normed and rotated at position *Pp + 1 + j
void launch_dr_qnorm(float* q, const float* qn, const float* cs, const float* sn, const int* Pp, int j, int hd,
                     hipStream_t st);
// a chain's inputs: in = {tok, P, hrow, _, h[1536]}; hin = h (hrow < 0) or hbase row hrow;
// tok[0] = tok; geo[2 j + s] = the attention geometry of step j on sliding (s = 0) / global layers
void launch_dr_setup(const int* in, const float* hbase, float* hin, int* tok, AttnGeom* geo, int k, int T,
                     hipStream_t st);
void launch_dr_rank(const float* score, int C, int* top, hipStream_t st);
void launch_dr_best(const float* cs, const int* top, const int* order, int nc, int* tok, int* sec, float* gap,
                    hipStream_t st);

// raw split-KV attention with explicit geometry (C-ABI entry point)
struct AttnGeom {
  int M, kmin, kmax, T;
  int pos[MAXM], lo[MAXM], skip_lo[MAXM], skip_hi[MAXM];
};
// E:1019-1059 alone: the merge of T splits' partials po [T][M][8][256], pm, pl (as k_attn_rows leaves
// them) into out [M][ldo]; with gs, out staged (staged_index) with its group sums [M][ldo / 32]
// xq / xqs not null (with gs): the rows also quantised for a W4A8 product, the four operand words of
// group g of row m at xq[(m * ldo / 32 + g) * 4] and its scale at xqs[m * ldo / 32 + g]
void launch_attn_merge(const float* po, const float* pm, const float* pl, int M, int T, float* out, int ldo,
                       float* gs, hipStream_t st, uint64_t* xq = nullptr, float* xqs = nullptr);
// nh query heads (a multiple of 2, at most 8) of q rows [M][ldq]; partials keep the 8-head layout
// gs not null: out written in the staged GEMV input layout (staged_index) with its group sums
// [M][ldo / 32]
void launch_attn_geom(const uint16_t* KC, const uint16_t* VC, const float* q, int ldq, const AttnGeom& g,
                      float* po, float* pm, float* pl, float* out, int ldo, hipStream_t st, int nh = NQ,
                      float* gs = nullptr);
// the same for head dim 512 (g4v_attn_hd.hip), 8 heads, partials [T][M][8][512]; out plain
// [M][ldo] or, with gs, staged (staged_index) with its group sums [M][ldo / 32].  Returns -1
// (nothing launched) for a shape it does not serve: a split longer than ATT_SPLIT_MAX keys.
constexpr int ATT_SPLIT_MAX = 4096;
int launch_attn_geom_hd(const uint16_t* KC, const uint16_t* VC, const float* q, int ldq, const AttnGeom& g, int hd,
                        float* po, float* pm, float* pl, float* out, int ldo, float* gs, hipStream_t st);
// head dim 512 with the geometry read from device memory (M rows, T splits and nh heads fixed by
// the launch; at most ATT_SPLIT_MAX keys per split, which the caller checks), out plain [M][ldo]
// or, with gs, staged with its group sums
void launch_attn_geom_dev_hd(const uint16_t* KC, const uint16_t* VC, const float* q, int ldq, const AttnGeom* gdev,
                             int M, int T, int nh, float* po, float* pm, float* pl, float* out, int ldo, hipStream_t st,
                             float* gs = nullptr, uint64_t* xq = nullptr, float* xqs = nullptr);
// the same with the geometry read from device memory (M rows and T splits fixed by the launch)
void launch_attn_geom_dev(const uint16_t* KC, const uint16_t* VC, const float* q, int ldq, const AttnGeom* gdev, int M,
                          int T, float* po, float* pm, float* pl, float* out, int ldo, hipStream_t st, int nh = NQ,
                          float* gs = nullptr, uint64_t* xq = nullptr, float* xqs = nullptr);
// E:1325-1326 the split geometry of a verify pass from its step parameters: geo[0] for the
// sliding-window layers, geo[1] for the global ones (window 512 from each row's RoPE position),
// T splits
void launch_step_geom(const StepDev* sp, int T, AttnGeom* geo, hipStream_t st);

}  // namespace g4v

namespace g4v {
// positions per attention split the split kernel can hold
int attn_pmax();
// device bandwidth probe (g4v_stream.hip): mode 0 reads src (one word per thread to dst, a sink
// of stream_grid() x 256 uint4), 1 copies src to dst, 2 fills dst with a pattern
int stream_grid();
void launch_stream(int mode, const uint4* src, uint4* dst, size_t n16, hipStream_t st);
// device [npos][256] key / value rows into the device cache layout (kv_cap(npos) positions)
void launch_kv_to_cache(const uint16_t* K, const uint16_t* V, int npos, uint16_t* KC, uint16_t* VC, hipStream_t st);
}
