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

// per-layer pointers for the layer kernels
struct LayerNorms {
  const float* in_ln;      // [H]
  const float* post_attn;  // [H]
  const float* pre_ff;     // [H]
  const float* post_ff;    // [H]
  const float* qn;         // [HD]
  const float* kn;         // [HD]
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

// synthetic weights (same formulas as the oracle's generator)
void launch_gen_bf16_normal(uint16_t* out, size_t n, uint64_t seed, float scale, hipStream_t st);
void launch_gen_w4(uint8_t* w, uint16_t* s, size_t nbytes, size_t nscales, uint64_t sw, uint64_t ss,
                   hipStream_t st);

// raw split-KV attention with explicit geometry (C-ABI entry point)
struct AttnGeom {
  int M, kmin, kmax, T;
  int pos[MAXM], lo[MAXM], skip_lo[MAXM], skip_hi[MAXM];
};
void launch_attn_geom(const uint16_t* KC, const uint16_t* VC, const float* q, int ldq, const AttnGeom& g,
                      float* po, float* pm, float* pl, float* out, int ldo, hipStream_t st);

}  // namespace g4v

namespace g4v {
// positions per attention split the split kernel can hold
int attn_pmax();
}
