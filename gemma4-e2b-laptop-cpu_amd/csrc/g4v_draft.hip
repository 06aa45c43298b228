// g4v_draft.hip -- prompt-lookup drafter over a token history kept on the device.
//
// Restates the prompt-lookup branch of run_req (E:1624-1628).  seq is the prompt followed by
// every committed token, L = |seq|.  With n > 0 and L > n, the drafts are the tokens that
// followed the most recent earlier occurrence of seq's last n tokens:
//   i* = max { i in [0, L-n-1] : seq[i .. i+n) == seq[L-n .. L) }
//   drafts = seq[i*+n .. min(i*+n+maxlen, L))
// and no drafts when no such i exists.  The reference scans i downwards and stops at the first
// hit; the maximum over all hits is the same index, so the scan runs in parallel here: one block
// tests CH candidates at a time, from the end of the history towards its start, and stops at the
// first chunk that holds a hit (the largest hit of that chunk, through an LDS atomicMax).
//
// The round's committed tokens come in by value and are written to the history by the same
// launch; every read of a position at or past the old length takes them from an LDS copy, so
// no thread reads a history word that this launch writes.
#include "g4v_internal.h"

namespace g4v {

namespace {

constexpr int PL_NT = 1024;     // threads of the one block
constexpr int PL_CPT = 4;       // candidates per thread and chunk
constexpr int PL_CH = PL_NT * PL_CPT;

__global__ __launch_bounds__(PL_NT) void k_prompt_lookup(int* __restrict__ hist, int L0, PlAppend app, int n,
                                                         int maxlen, int* __restrict__ out) {
  __shared__ int tail[PL_MAXN];
  __shared__ int added[PL_MAXA];
  __shared__ int best;
  const int tid = threadIdx.x;
  const int L = L0 + app.n;
  auto tok = [&](int p) -> int { return p >= L0 ? added[p - L0] : hist[p]; };
  if (tid < app.n) {
    added[tid] = app.t[tid];
    hist[L0 + tid] = app.t[tid];
  }
  if (tid == 0) best = -1;
  __syncthreads();
  const bool look = n > 0 && L > n;  // E:1624,1626: NG_N > 0 and L > NG_N
  if (look)
    for (int t = tid; t < n; t += PL_NT) tail[t] = tok(L - n + t);
  __syncthreads();
  // candidates i = top - c for c in [0, top]; chunk q covers c in [q*CH, (q+1)*CH)
  const int top = look ? L - n - 1 : -1;
  for (int c0 = 0; c0 <= top; c0 += PL_CH) {
#pragma unroll
    for (int r = 0; r < PL_CPT; ++r) {
      const int i = top - (c0 + r * PL_NT + tid);
      if (i < 0) break;
      bool eq = true;
      for (int t = 0; t < n; ++t)
        if (tok(i + t) != tail[t]) {
          eq = false;
          break;
        }
      if (eq) atomicMax(&best, i);
    }
    __syncthreads();
    if (best >= 0) break;  // uniform: every thread reads the value the barrier published
    __syncthreads();       // no thread's next-chunk atomic may precede another's read above
  }
  const int b = best;
  const int nd = b < 0 ? 0 : min(maxlen, L - b - n);
  if (tid < nd) out[1 + tid] = tok(b + n + tid);
  if (tid == 0) out[0] = nd;
}

}  // namespace

void launch_prompt_lookup(int* hist, int L0, const PlAppend& app, int n, int maxlen, int* out, hipStream_t st) {
  hipLaunchKernelGGL(k_prompt_lookup, dim3(1), dim3(PL_NT), 0, st, hist, L0, app, n, maxlen, out);
}

}  // namespace g4v
