// g4v_head.h -- device data of the certified head (screen + exact rescore + argmax).
#pragma once
#include "g4v_internal.h"

namespace g4v {

// exp3 head expanded to its decoded bf16 weights plus the exception list (CSR by row)
struct HeadDev {
  const uint4* dec;      // [V][24][8] uint4: lane j of group pair p: w[j],w[16+j],w[8+j],w[24+j] x2
  uint4* decw;           // writable alias used while building
  const int* exc_ptr;    // [V+1]
  const uint16_t* exc_col;
  const float* exc_del;
  uint16_t* exc_col_w;   // writable aliases used while building
  float* exc_del_w;
  const uint8_t* cb;     // [8] exponent codebook (device)
  // the exp3 form streamed by the full head (X3:1-4 packing, laid out for the lane order of
  // dec): per (row, group pair p, lane j) the sign|mantissa bytes of dec's 8 weights w0..w7 as
  // {w0 w2 w4 w6 | w1 w3 w5 w7} and their codebook indices, byte b = idx(w_2b) | idx(w_2b+1) << 4
  const uint2* x3sm;     // [V][24][8]
  const uint32_t* x3ix;  // [V][24][8]
  uint2* x3smw;          // writable aliases used while building
  uint32_t* x3ixw;
};

// per-call scratch for up to MAXM rows
struct HeadScratch {
  float* u;          // [MAXM][V]: U bounds, then full-head logits of fallback rows
  int* list;         // [MAXM][HEAD_LIMIT] survivor indices (unordered)
  float* sval;       // [MAXM][HEAD_LIMIT] rescored r16 logits
  int* cnt;          // [MAXM] survivor count (may exceed the limit)
  int32_t* lmax_key; // [MAXM] fkey(max L)
  int32_t* vmax_key; // [MAXM] fkey(max rescored logit)
  int* best;         // [MAXM] greedy token (lowest index of the tie set)
  float* thr;        // [MAXM] calc_thr(max L)
  float* lpart;      // [MAXM][HEAD_MAXGRID] per-block max of L from the screen
  float* vpart;      // [MAXM][HEAD_MAXGRID] per-block max logit of the full head
};
constexpr int HEAD_MAXGRID = 4096;

struct HeadBuildTmp {
  unsigned long long* hist;  // [256]
  uint8_t* gcnt;             // [V][48]
  int* rowcnt;               // [V]
};

// optional hook around each launch (per-kernel-class HIP-event timing in the C ABI)
struct ProfHook {
  void (*mark)(void* ctx, int tag, int begin, double bytes) = nullptr;
  void* ctx = nullptr;
};
enum ProfTag {
  PT_GEMV_QKV = 0, PT_GEMV_O, PT_GEMV_GATEUP, PT_GEMV_DOWN, PT_ATTN, PT_ROWS, PT_HEAD_SCREEN, PT_HEAD_SELECT,
  PT_HEAD_RESCORE, PT_HEAD_FULL, PT_HEAD_TIE, PT_ACCEPT, PT_HEAD2, PT_NTAGS
};

struct HeadRun {
  ProfHook prof;
  double full_bytes;     // algorithmic bytes of one full-head pass (for the hook)
  int pass2;             // 1: second head pass of a verify step
  HeadScratch hs;
  HeadDev hd;
  W4Dev screen;
  const float* coef;
  const uint16_t* lut;   // cap LUT over bf16 inputs
  const float* h;        // [MT][H] final-normed rows (bf16-valued)
  const float* hn;       // [MT] (float)sqrt(sum h^2)
  const int* active;     // optional device flag: 0 -> nothing runs
  int MT, V, grid_cap;
};

void head_build(const uint16_t* E, int V, HeadDev& hd, HeadBuildTmp& tmp, hipStream_t st);
void head_build_dec(const uint16_t* E, int V, HeadDev& hd, HeadBuildTmp& tmp, hipStream_t st);
void head_build_exc(const uint16_t* E, int V, HeadDev& hd, hipStream_t st);
void head_build_x3(int V, HeadDev& hd, hipStream_t st);
void screen_build(const uint16_t* E, int V, uint8_t* Wq, uint16_t* Sq, float* coef, hipStream_t st);
void head_run(const HeadRun& r, hipStream_t st);
size_t head_lds(int MT);

}  // namespace g4v
