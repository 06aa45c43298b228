// g4v_internal.h -- device-side data structures and kernel launchers shared by the
// translation units of libg4v.  Not part of the C ABI (include/g4v.h is).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

#include "g4v_num.h"

namespace g4v {

constexpr int H = 1536;       // hidden size
constexpr int HD = 256;       // head dim
constexpr int NQ = 8;         // query heads (one KV head)
constexpr int MAXM = 8;       // rows per verify pass
constexpr int MAXT = 16;      // split-KV splits

// Device KV cache layout (per layer: positions 0 .. kvcap - 1, kvcap a multiple of 32).
// Keys: a position's 256 values in chain-lane order -- element e = 16 tt + 8 s + l (the
// reference's score lane l, chain s, step tt) at slot l * 32 + s * 16 + tt -- so that the 8
// lanes scoring one position each read 64 contiguous bytes.  Values: blocks of 32 positions in
// four parts of 8 positions, each part dim-major (8 values of a dim = 16 bytes), so that the
// lane of dim i reads part c of a block as 16 bytes and a wave's 64 lanes read one part of 64
// dims as 1 KB in one contiguous load.  Both are permutations of the reference's [position][256]
// rows.
__host__ __device__ inline int kc_slot(int e) { return (e & 7) * 32 + ((e >> 3) & 1) * 16 + (e >> 4); }
__host__ __device__ inline size_t kc_index(int p, int e) { return (size_t)p * HD + kc_slot(e); }
__host__ __device__ inline size_t vc_index(int p, int i) {
  return (size_t)(p >> 5) * (32 * HD) + (size_t)((p >> 3) & 3) * (8 * HD) + (size_t)i * 8 + (p & 7);
}
inline int kv_cap(int npos) { return (npos + 31) / 32 * 32; }  // positions of a layer's cache slab
// the same layouts for a head dim D (256 or 512: the global layers of the Gemma-4-E2B layout).
// Keys, D = 256: as above.  D = 512: element e = 16 tt + 8 s + l (tt < 32) at slot
// 64 (4 s + tt / 8) + 8 l + tt % 8, i.e. lane l's k-th 16 bytes (k = 4 s + tt / 8, the 8 steps
// tt of chain s from 8 (k % 4)) are 16-byte word 8 k + l of the row: the 8 lanes scoring a
// position read 128 contiguous bytes per load, 8 loads a row.  In both, the 8 steps of a chain
// from a multiple of 8 are 8 contiguous slots.
template <int D>
__host__ __device__ inline int kc_slot_d(int e) {
  if constexpr (D == 512)
    return (4 * ((e >> 3) & 1) + (e >> 7)) * 64 + (e & 7) * 8 + ((e >> 4) & 7);
  else
    return (e & 7) * (D / 8) + ((e >> 3) & 1) * (D / 16) + (e >> 4);
}
template <int D>
__host__ __device__ inline size_t kc_index_d(int p, int e) { return (size_t)p * D + kc_slot_d<D>(e); }
template <int D>
__host__ __device__ inline size_t vc_index_d(int p, int i) {
  return (size_t)(p >> 5) * (32 * D) + (size_t)((p >> 3) & 3) * (8 * D) + (size_t)i * 8 + (p & 7);
}
constexpr int HEAD_LIMIT = 30000;  // E:1416 LIM: more survivors -> full head

// An int4 G32 matrix on the device.  wr: weights re-laid for the exact-order GEMV
// (row n, chunk c of 8 groups, lane j: 16 bytes = bytes j and 8+j of each group);
// s: bf16 scales in the reference's [N][K/32] layout.
struct W4Dev {
  const uint4* wr;
  const uint16_t* s;
  int N, K;
};

// Where the GEMV epilogue sends the result.
enum GemvEpi { EPI_STORE = 0, EPI_GATEUP = 1, EPI_SCREEN = 2 };

// Staged activation layout of a K-vector.  Lane j (0..7) of a W4G32 chain multiplies, in
// group g, the four values x[32g+2j], x[32g+16+2j], x[32g+2j+1], x[32g+17+2j]; the staged
// row stores them as one float4 at float4 index 8g + j, so a GEMV stages its activations with
// straight 16-byte copies.  Rows of M vectors follow each other (K floats per row).  The
// per-group sums (sequential fp32 sum of x[32g..32g+31], W:22) travel beside it as [M][K/32].
__host__ __device__ __forceinline__ int staged_index(int n) {
  const int g = n >> 5, i = n & 31, e = i & 15;
  return (g * 8 + (e >> 1)) * 4 + ((e & 1) ? 2 : 0) + (i >> 4);
}

// Range-checked 16-byte loads through a buffer resource: a lane whose offset lies past the
// resource's num_records bytes reads zeros and moves no data (a stream reads exactly its range,
// without clamped duplicate fetches).  The base must be uniform over the wave.  Being intrinsic
// calls rather than plain loads, a ring of them carried across a loop's back edge stays a ring
// (plain loads there get folded into loads at the top of the next iteration).
// quant of one 32-group (engine/w4a8_avx2.h:33-41) into its four operand words.  q = RNE(x * inv)
// clamped to [-128, 127] is formed as y = med3(x * inv, -128, 127) + 1.5 * 2^23: the add rounds to
// the nearest integer, ties to even (the ulp there is 1), as cvtps_epi32 does in the default mode,
// and clamping before rounding gives the same integer (the bounds are integers, rounding is
// monotonic); the low byte of y's bits is then q in two's complement.
__device__ __forceinline__ float a8_quant_group(const float (&v)[32], uint64_t (&aq)[4]) {
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
  const float sx = amax / 127.0f, inv = sx > 0.f ? 1.0f / sx : 0.0f;
  uint32_t qb[32];
#pragma unroll
  for (int i = 0; i < 32; ++i)
    qb[i] = __float_as_uint(__builtin_amdgcn_fmed3f(v[i] * inv, -128.0f, 127.0f) + 12582912.0f);
  // operand word h: low dword elements 8h + 0, 2, 4, 6, high dword 8h + 1, 3, 5, 7 (low bytes)
  auto pack4 = [](uint32_t a, uint32_t b, uint32_t c, uint32_t d) -> uint32_t {
    return __builtin_amdgcn_perm(b, a, 0x0c0c0400u) | (__builtin_amdgcn_perm(d, c, 0x0c0c0400u) << 16);
  };
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const uint32_t* q = qb + 8 * h;
    aq[h] = (uint64_t)pack4(q[0], q[2], q[4], q[6]) | ((uint64_t)pack4(q[1], q[3], q[5], q[7]) << 32);
  }
  return sx;
}

// A block barrier that orders LDS only: each wave's LDS operations complete before it, while
// its global loads stay in flight across it (__syncthreads' workgroup fence also waits for every
// outstanding global load, so register prefetches issued before it would all land there).  For
// blocks whose waves exchange data through LDS alone.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  uint4 u;
  __builtin_memcpy(&u, &v, 16);
  return u;
}

// lane n of a 16-lane row takes lane n + N of the row (row_shl:N; lanes past the row get 0)
template <int N>
__device__ __forceinline__ float shl_f(float v) {
#if defined(__HIP_DEVICE_COMPILE__)
  return as_f32((uint32_t)__builtin_amdgcn_update_dpp(0, (int)as_u32(v), 0x100 + N, 0xF, 0xF, false));
#else
  return v;
#endif
}
template <int N>
__device__ __forceinline__ double shl_d(double v) {
#if defined(__HIP_DEVICE_COMPILE__)
  const uint64_t u = as_u64(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, 0x100 + N, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), 0x100 + N, 0xF, 0xF, false);
  return as_f64(((uint64_t)hi << 32) | lo);
#else
  return v;
#endif
}
// lane 0 of each 16-lane row to the whole row (row_newbcast:0)
__device__ __forceinline__ double bcast0_d(double v) {
#if defined(__HIP_DEVICE_COMPILE__)
  const uint64_t u = as_u64(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, 0x150, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), 0x150, 0xF, 0xF, false);
  return as_f64(((uint64_t)hi << 32) | lo);
#else
  return v;
#endif
}

// ---- operands broadcast within rows of 16 lanes (DPP row_newbcast) ----
// A VGPR whose lane k (of every row of 16 lanes) holds value k serves 16 wave-uniform operands:
// the instruction reads lane k of its row.  The source registers of these are written by LDS or
// memory loads only, never by a VALU instruction just before (the DPP read-after-VALU-write hazard).
// d = x[k] * w
template <int K>
__device__ __forceinline__ float mul_bc(float x, float w) {
#if defined(__HIP_DEVICE_COMPILE__)
  float d;
  asm("v_mul_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf" : "=v"(d) : "v"(x), "v"(w), "n"(K));
  return d;
#else
  return x * w;
#endif
}
// o = w[k] * v + o
template <int K>
__device__ __forceinline__ float fmac_bc(float o, float w, float v) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf" : "+v"(o) : "v"(w), "v"(v), "n"(K));
  return o;
#else
  return fmaf(w, v, o);
#endif
}
// l = l + w[k]
template <int K>
__device__ __forceinline__ float add_bc(float l, float w) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm("v_add_f32_dpp %0, %1, %0 row_newbcast:%2 row_mask:0xf bank_mask:0xf" : "+v"(l) : "v"(w), "n"(K));
  return l;
#else
  return l + w;
#endif
}
// f(integral_constant<int, k>) for k = 0 .. N-1, each k a compile-time constant
template <typename F, int... K>
__device__ __forceinline__ void unroll_impl(F& f, std::integer_sequence<int, K...>) {
  (f(std::integral_constant<int, K>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void unroll_n(F& f) {
  unroll_impl(f, std::make_integer_sequence<int, N>{});
}

// The 16-lane head order of a 256-wide head: element e = 16 tt + n at n * 16 + tt, so that lane n
// of a row of 16 lanes reads its 16 elements (its sum-of-squares lane, score chain and RoPE
// pairs, tt and tt + 8) as four 16-byte words.  Applied per head of 256 to wider rows.
__host__ __device__ __forceinline__ int head16_index(int e) {
  return (e & ~255) | ((e & 15) << 4) | ((e >> 4) & 15);
}

struct GemvArgs {
  W4Dev mat[3];       // up to three matrices with the same K, processed in one launch
  float* y[3];        // outputs [M][ldy]
  int ldy[3];
  int tiles[4];       // prefix sum of 32-row tiles per matrix
  const float* x;     // activations [M][ldx] (plain layout), or
  const float4* xs;   // activations [M][K/4] in the staged layout (used when not null)
  const float* gs;    // their group sums [M][K/32] (computed in LDS when null)
  int ldx;
  int K;
  int kphase;         // K elements staged in LDS at a time (set by launch_gemv)
  int lds_budget;     // LDS bytes a block may stage (0: 64 KB)
  int y_staged;       // EPI_GATEUP: write the activation in the staged layout (ldy = row length)
  int M;              // runtime rows (<= template MT); rows >= M are not computed
  // EPI_SCREEN
  const float* coef;  // [N]
  const float* hn;    // [MT]
  float* lpart;       // [MT][gridDim.x] per-block max of L (reduced by the consumer)
  const int* active;  // optional: a device count; 0 -> the launch does nothing
};

void launch_relayout_w4(const uint8_t* w, uint4* wr, int N, int K, hipStream_t st);

// Row-tiled copy of a re-laid matrix for the row-tile GEMV (g4v_gemvt.hip): N a multiple of 64;
// w: [N/64][K/256][8][64] uint4, the chunk (c, j) of the tile's 64 rows contiguous (one 1 KB
// wave load); s: [N/64][K/256][64] uint4, the 8 bf16 scales of chunk c of each row.
struct W4Tile {
  const uint4* w;
  const uint4* s;
  int N;
};
void launch_tile_w4(const uint4* wr, const uint16_t* s, uint4* tw, uint4* ts, int N, int K, hipStream_t st);
// gate / up pair of N rows each: 64-row tile t holds pairs 32t..32t+31 as 16 gate rows, their 16
// up rows, the next 16 gate rows and their 16 up rows
void launch_tile_w4_pair(const uint4* wg, const uint16_t* sg, const uint4* wu, const uint16_t* su, uint4* tw,
                         uint4* ts, int N, int K, hipStream_t st);

// Row-tile GEMV: y[mi][m][n] for up to three matrices with the same K (N multiples of 64),
// activations in the staged layout with optional group sums (formed in LDS when null).  With
// gateup set, mat[0] is a gate / up pair (launch_tile_w4_pair, N rows each) and y[0] receives
// the activation gelu(gate) * up of each of the N rows, in the staged layout (row length ldy[0]).
struct GemvTArgs {
  W4Tile mat[3];
  float* y[3];
  int ldy[3];
  const float4* xs;  // [M][K/4] staged
  const float* gs;   // [M][K/32] or null
  int K;
  int M;
  int gateup;
  // merge prologue (mrg_po not null, K = NQ * HD, xs / gs unused): the activations are the
  // split-KV merge (E:1019-1059) of the attention partials po [T][M][NQ][HD], pm / pl
  // [T][M][NQ], formed by every block for its own rows
  const float* mrg_po;
  const float* mrg_pm;
  const float* mrg_pl;
  int mrg_T;
  // norm prologue (nrm_mode != 0, K = H, xs / gs unused): the block forms its rows' activations
  // from the previous sub-block's output o and the residual stream xin:
  //   x1 = r16(xin + r16((r16(o) * r1) * w1)), mode 2 (after the MLP) then x1 = r16(x1 * scalar);
  //   xa = (x1 * r2) * w2, rounded to bf16 in mode 1 (after attention);
  // r1, r2 the RMS factors of r16(o) and x1.  The blocks of tile 0 write x1 to xout (a buffer
  // other than xin, which the other blocks still read).
  int nrm_mode;
  const float* nrm_o;
  const float* nrm_xin;
  float* nrm_xout;
  const float* nrm_w1;
  const float* nrm_w2;
  float nrm_scalar;
  // the per-layer-input gate of the Gemma-4-E2B layout (E:1375-1386, pg_fused_task E:405-443):
  // with epi_pli set, the norm prologue stops at x1 (mode 3: the MLP residual without scalar or
  // second norm, x1 the product's input) and the output is g2 = r16(r16(gelu8(r16 y)) *
  // r16(epi_pli[m * epi_pli_ld + n])), written staged into y[0] ([M][ldy]) for the next product
  const float* epi_pli;
  int epi_pli_ld;
  // bit mi set: matrix mi's outputs are written in the 16-lane head order (head16_index), the
  // order the verify pass's attention reads its query, key and value rows in
  int yperm;
  // W4A8 products (launch_gemv_a8): xq / xqs, the staged rows already quantised (operand words
  // [M][K/32][4], scales [M][K/32]) in place of xs; yq / yqs (gate / up of the 6144-wide MLP): the
  // activation also quantised, group c of row m at yq[(m * N / 32 + c) * 4] and yqs[m * N / 32 + c]
  const uint64_t* xq;
  const float* xqs;
  uint64_t* yq;
  float* yqs;
};
// W4A8 (g4v_w4a8.hip): operand tiles of a matrix from its original bytes [N][K/2] and scales
// [N][K/32] (N % 16 == 0): tw [N/16][K/128][64] uint4, ts [N/16][K/256][16] uint4
void launch_tile_a8(const uint8_t* w, const uint16_t* s, uint4* tw, uint4* ts, int N, int K, hipStream_t st);
// quantised rows: xqb [Mpad][K] bf16 (MFMA operand order), sxt / corr [K/32][Mpad]; q / sx / sum
// (optional, plain layouts [M][K], [M][K/32]) for the quant entry point
void launch_w4a8_quant(const float* x, int M, int Mpad, int K, uint16_t* xqb, float* sxt, float* corr, int8_t* qo,
                       float* sxo, int32_t* sumo, hipStream_t st);
// W4A8 products of decode rows (M <= 8) over up to three matrices of one input (N_j % 16 == 0):
// matrix j's tiles are blocks t0[j] .. t0[j + 1] - 1; t0[j] = t0[n] for j >= n.
struct A8Dec {
  const uint4* tw[3];
  const uint4* ts[3];
  float* y[3];
  int ldy[3];
  int t0[4];
};
int launch_w4a8_dec(const A8Dec& m, int n, const uint16_t* xqb, const float* sxt, const float* corr, int M, int K,
                    hipStream_t st);
void launch_w4a8_gemm(const uint4* tw, const uint4* ts, const uint16_t* xqb, const float* sxt, const float* corr,
                      float* y, int M, int N, int K, int ldy, hipStream_t st);
int w4a8_mpad(int M);  // rows the quantised operand holds for M rows

// prompt lookup (g4v_draft.hip): appends app.t[0 .. app.n) to hist [L0 ..] and writes
// out[0] = draft count, out[1 ..] = drafts (n <= PL_MAXN, n + 1 <= L0 + app.n, maxlen <= PL_MAXD)
constexpr int PL_MAXA = 16, PL_MAXN = 256, PL_MAXD = 16;
struct PlAppend {
  int n;
  int t[PL_MAXA];
};
void launch_prompt_lookup(int* hist, int L0, const PlAppend& app, int n, int maxlen, int* out, hipStream_t st);

// mpl: activation rows per block (1..4, 2 at most with the merge prologue); tr: rows per tile
// (64 or 32).  Returns the grid size (0: K unsupported, nothing launched).
int launch_gemv_t(const GemvTArgs& a, hipStream_t st, int mpl, int tr);
// W4A8 products of a verify pass (g4v_gemva8.hip): the same arguments with mat[j] the a8 tiles
// (launch_tile_a8) and, with gateup set, mat[0] / mat[1] the gate / up matrices; M <= 8, the
// staged input xs (quantised in the product's blocks) or a norm prologue (modes 1 and 2, or 3
// with epi_pli).  Returns the grid size of the product (0: refused, nothing launched).
int launch_gemv_a8(const GemvTArgs& a, hipStream_t st);
// whether launch_gemv_a8's gate / up launch of N pairs honours yq / yqs (four tiles a block: each
// block owns one 32-group of every row)
inline bool a8_gateup_quantises(int N) { return N % 32 == 0; }
// returns the grid size used (the number of EPI_SCREEN partials per activation row)
int launch_gemv(const GemvArgs& a, int epi, hipStream_t st, int grid_cap = 0);
// grid launch_gemv would use
int gemv_grid(const GemvArgs& a, int epi, int grid_cap);

}  // namespace g4v
