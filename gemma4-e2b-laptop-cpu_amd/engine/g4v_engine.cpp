// g4v_engine.cpp -- the engine's process boundary over the gfx950 library: the same command line
// and line protocol as the reference engine (engine/gemma4_engine.cpp, cited as E), so that a
// front-end written for it (its server, bench scripts) drives the GPU path unchanged.
//
//   g4v_engine <model> <index> <prompt.ids> <nnew>          one request (E:1211, 1689)
//   ENGINE_SERVE=1 g4v_engine <model> <index> - 0           requests on stdin (E:1681-1688):
//     "N id id ..."  -> FIRST <id> after the prefill, TOK <ids> per round (ENGINE_STREAM), then
//                       GEN: <ids> and a TIMING line (E:1604, 1612-1614, 1672-1679)
//     "BENCH_MODE k tree" -> MODE k=.. tree=.. / MODE_ERROR (E:1683)
//
// <model> is a checkpoint directory holding model.safetensors and <index> its tensor index (one
// line per tensor: name, dtype, byte offset in the file, byte count, shape; E:1218-1222), or
// "synth:SEED:V:NL:I" for the synthetic stack (<index> ignored).  A checkpoint holding the
// per-layer-input tensors is the Gemma-4-E2B layout main() loads (E:1222-1231: 35 layers of head
// dim 256 / 512, k/v projections in layers 0..14, per-layer MLP widths, the per-layer embedding
// table) and runs through g4v_model_create_gemma; its MTP drafter is the drafter checkpoint
// main() loads with ENGINE_K > 0 (ENGINE_DRAFTER_DIR / ENGINE_DRAFTER_INDEX, E:1519-1528).  Any other checkpoint is read as a uniform stack: every layer with its
// own q/k/v projections of 8 x 256 / 256 / 256 rows and one MLP width.  The MTP drafter is the
// synthetic one (ENGINE_DRAFTER_SEED; with a uniform checkpoint only when set).  run_req (E:1584-1676) is restated over the C ABI: the prefix cache
// (g4v_slot_*), the prefill (g4v_prefill), and decode rounds whose drafts come from prompt
// lookup (ENGINE_NGRAM / ENGINE_NGLEN) or, when it finds none, the MTP drafter (ENGINE_K, a
// synthetic drafter, seed ENGINE_DRAFTER_SEED), verified as a chain (g4v_verify_step) or, when
// the drafter's runner-up is proposed as a sibling row (E:1634-1655: ENGINE_SIB_GAP,
// ENGINE_SIB_LONG, ENGINE_TREE / BENCH_MODE k 1, ENGINE_POLICY), with g4v_verify_sibling.
// Prompt-lookup drafts of a round are capped at 4 (the verify step's chain).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/g4v.h"

namespace {

g4v_ctx* G = nullptr;

void check(int rc, const char* what) {
  if (rc != 0) {
    fprintf(stderr, "g4v %s: %s (%d)\n", what, g4v_error(G), rc);
    fflush(stderr);
    exit(1);
  }
}

int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v ? atoi(v) : dflt;
}

bool is_stop(int t) { return t == 106 || t == 1; }  // E:1609

constexpr int ATT_PAR = 192;  // E:1214

// ---- checkpoint (E:147-175, 1218-1231) ----
struct Tensor {
  std::string dtype;
  size_t off = 0, nbytes = 0;
  std::vector<long long> shape;
};

struct Checkpoint {
  std::map<std::string, Tensor> idx;
  const uint8_t* base = nullptr;
  size_t size = 0;

  [[noreturn]] static void fail(const std::string& m) {
    fprintf(stderr, "checkpoint: %s\n", m.c_str());
    exit(2);
  }
  void open_files(const std::string& dir, const std::string& index) {
    std::ifstream f(index);
    if (!f) fail("cannot read index " + index);
    std::string line;
    while (std::getline(f, line)) {  // name \t dtype \t offset \t nbytes \t shape (comma separated)
      std::stringstream ss(line);
      std::string n, d, o, b, sh;
      if (!std::getline(ss, n, '\t') || !std::getline(ss, d, '\t') || !std::getline(ss, o, '\t') ||
          !std::getline(ss, b, '\t'))
        continue;
      std::getline(ss, sh, '\t');
      Tensor t;
      t.dtype = d;
      t.off = std::stoull(o);
      t.nbytes = std::stoull(b);
      std::stringstream s2(sh);
      std::string x;
      while (std::getline(s2, x, ',')) t.shape.push_back(std::stoll(x));
      idx[n] = t;
    }
    const std::string path = dir + "/model.safetensors";
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) fail("cannot open " + path);
    struct stat st;
    fstat(fd, &st);
    size = (size_t)st.st_size;
    void* p = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (p == MAP_FAILED) fail("cannot map " + path);
    base = (const uint8_t*)p;
  }
  // E:170: the language model's prefix first
  const Tensor* find(const std::string& n) const {
    auto it = idx.find("model.language_model." + n);
    if (it == idx.end()) it = idx.find(n);
    return it == idx.end() ? nullptr : &it->second;
  }
  const Tensor& get(const std::string& n, const char* dtype, size_t nbytes) const {
    const Tensor* t = find(n);
    if (!t) fail("missing tensor " + n);
    if (t->dtype != dtype) fail(n + ": dtype " + t->dtype + ", expected " + dtype);
    if (t->nbytes != nbytes) fail(n + ": " + std::to_string(t->nbytes) + " bytes, expected " + std::to_string(nbytes));
    if (t->off + t->nbytes > size) fail(n + ": beyond the end of the file");
    return *t;
  }
  const uint8_t* data(const Tensor& t) const { return base + t.off; }
  std::vector<float> vec(const std::string& n, size_t len) const {  // bf16 vector widened (E:172)
    const Tensor& t = get(n, "BF16", len * 2);
    std::vector<float> v(len);
    const uint16_t* p = (const uint16_t*)data(t);
    for (size_t i = 0; i < len; ++i) {
      const uint32_t u = (uint32_t)p[i] << 16;
      std::memcpy(&v[i], &u, 4);
    }
    return v;
  }
};

// an int4 G32 matrix (E:175): [N][K/8] int32 words = [N][K/2] bytes, bf16 scales [N][K/32]
void set_q4(const Checkpoint& ck, int l, int j, const std::string& b, int N, int K) {
  const Tensor* w = ck.find(b + ".weight_packed");
  if (w && w->shape.size() == 2 && (w->shape[0] != N || w->shape[1] * 8 != K))
    Checkpoint::fail(b + ": shape " + std::to_string(w->shape[0]) + " x " + std::to_string(w->shape[1] * 8) +
                     ", expected " + std::to_string(N) + " x " + std::to_string(K));
  const Tensor& wt = ck.get(b + ".weight_packed", "I32", (size_t)N * K / 2);
  const Tensor& st = ck.get(b + ".weight_scale", "BF16", (size_t)N * (K / 32) * 2);
  check(g4v_model_set_matrix(G, l, j, ck.data(wt), (const uint16_t*)ck.data(st)), "model_set_matrix");
}

// main()'s layout (E:1222-1231) into the library (g4v_model_create_gemma + setters)
void load_gemma(const Checkpoint& ck, int V, int ctx) {
  const int H = 1536, NL = 35, PD = 256;
  if (ck.find("layers.35.input_layernorm.weight") || !ck.find("layers.34.input_layernorm.weight"))
    Checkpoint::fail("the per-layer-input layout has 35 layers (E:1222)");
  std::vector<int> mlp(NL);
  for (int l = 0; l < NL; ++l) {
    const Tensor* g = ck.find("layers." + std::to_string(l) + ".mlp.gate_proj.weight_packed");
    if (!g || g->shape.size() != 2) Checkpoint::fail("layers." + std::to_string(l) + ".mlp.gate_proj missing");
    mlp[l] = (int)g->shape[0];
  }
  check(g4v_model_create_gemma(G, V, mlp.data(), ctx), "model_create_gemma");
  check(g4v_model_set_embed(G, (const uint16_t*)ck.data(ck.get("embed_tokens.weight", "BF16", (size_t)V * H * 2))),
        "model_set_embed");
  const char* names[9] = {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                          "mlp.gate_proj",    "mlp.up_proj",      "mlp.down_proj",    "per_layer_input_gate",
                          "per_layer_projection"};
  for (int l = 0; l < NL; ++l) {  // E:1224-1229
    const std::string p = "layers." + std::to_string(l) + ".";
    const int hd = l % 5 != 4 ? 256 : 512, I = mlp[l];
    const bool owner = l < 15;
    const int Ns[9] = {8 * hd, hd, hd, H, I, I, H, PD, H}, Ks[9] = {H, H, H, 8 * hd, H, H, I, H, PD};
    for (int j = 0; j < 9; ++j)
      if (owner || (j != 1 && j != 2)) set_q4(ck, l, j, p + names[j], Ns[j], Ks[j]);
    std::vector<float> nv[7] = {ck.vec(p + "input_layernorm.weight", H), ck.vec(p + "post_attention_layernorm.weight", H),
                                ck.vec(p + "pre_feedforward_layernorm.weight", H),
                                ck.vec(p + "post_feedforward_layernorm.weight", H),
                                ck.vec(p + "post_per_layer_input_norm.weight", H), ck.vec(p + "self_attn.q_norm.weight", hd)};
    if (owner) nv[6] = ck.vec(p + "self_attn.k_norm.weight", hd);
    const float* nvp[7] = {nv[0].data(), nv[1].data(), nv[2].data(), nv[3].data(), nv[4].data(), nv[5].data(),
                           owner ? nv[6].data() : nullptr};
    check(g4v_model_set_norms_gemma(G, l, nvp, ck.vec(p + "layer_scalar", 1)[0]), "model_set_norms_gemma");
  }
  {  // E:1230-1231: the projection, its norm and the table (uploaded in slices of the mapped file)
    const int N = NL * PD;
    const Tensor& wt = ck.get("per_layer_model_projection.weight_packed", "I32", (size_t)N * H / 2);
    const Tensor& st = ck.get("per_layer_model_projection.weight_scale", "BF16", (size_t)N * (H / 32) * 2);
    check(g4v_model_set_ple(G, ck.data(wt), (const uint16_t*)ck.data(st),
                            ck.vec("per_layer_projection_norm.weight", PD).data()),
          "model_set_ple");
    const Tensor& tb = ck.get("embed_tokens_per_layer.weight", "BF16", (size_t)V * N * 2);
    const uint16_t* rows = (const uint16_t*)ck.data(tb);
    for (int t0 = 0; t0 < V; t0 += 8192)
      check(g4v_model_set_ple_rows(G, t0, std::min(8192, V - t0), rows + (size_t)t0 * N), "model_set_ple_rows");
  }
  check(g4v_model_set_final_norm(G, ck.vec("norm.weight", H).data()), "model_set_final_norm");
}

// E:1519-1528: the drafter checkpoint (bf16 tensors, the token ordering int64) into the library
void load_drafter(const Checkpoint& dk) {
  const int DH = 256, H = 1536, F = 2048;
  const Tensor* ce = dk.find("masked_embedding.centroids.weight");
  const Tensor* em = dk.find("model.embed_tokens.weight");
  if (!ce || ce->shape.size() != 2 || !em || em->shape.size() != 2)
    Checkpoint::fail("drafter: masked_embedding.centroids.weight / model.embed_tokens.weight missing");
  const int C = (int)ce->shape[0], V = (int)em->shape[0];
  auto bf = [&](const std::string& n, size_t count) {
    return (const uint16_t*)dk.data(dk.get(n, "BF16", count * 2));
  };
  g4v_drafter_tensors t{};
  t.C = C;
  t.pre = bf("pre_projection.weight", (size_t)DH * 2 * H);
  t.post = bf("post_projection.weight", (size_t)H * DH);
  t.cent = bf("masked_embedding.centroids.weight", (size_t)C * DH);
  t.emb = bf("model.embed_tokens.weight", (size_t)V * DH);
  t.norm = bf("model.norm.weight", DH);
  t.order = (const int64_t*)dk.data(dk.get("masked_embedding.token_ordering", "I64", (size_t)V * 8));
  const char* nn[5] = {"input_layernorm", "post_attention_layernorm", "pre_feedforward_layernorm",
                       "post_feedforward_layernorm", "self_attn.q_norm"};
  for (int l = 0; l < 4; ++l) {
    const std::string p = "model.layers." + std::to_string(l) + ".";
    const Tensor* q = dk.find(p + "self_attn.q_proj.weight");
    if (!q || q->shape.size() != 2) Checkpoint::fail("drafter: " + p + "self_attn.q_proj.weight missing");
    const int hd = (int)q->shape[0] / 4;
    t.hd[l] = hd;
    t.q[l] = bf(p + "self_attn.q_proj.weight", (size_t)4 * hd * DH);
    t.o[l] = bf(p + "self_attn.o_proj.weight", (size_t)DH * 4 * hd);
    t.gate[l] = bf(p + "mlp.gate_proj.weight", (size_t)F * DH);
    t.up[l] = bf(p + "mlp.up_proj.weight", (size_t)F * DH);
    t.down[l] = bf(p + "mlp.down_proj.weight", (size_t)DH * F);
    for (int k = 0; k < 5; ++k) t.nv[l][k] = bf(p + nn[k] + ".weight", k < 4 ? DH : hd);
    t.scalar[l] = bf(p + "layer_scalar", 1)[0];
  }
  check(g4v_drafter_load(G, &t), "drafter_load");
}

// the stack of a checkpoint into the library (g4v_model_create + setters); returns V
int load_checkpoint(const Checkpoint& ck, int ctx, bool* gemma) {
  const int H = 1536;
  const Tensor* emb = ck.find("embed_tokens.weight");
  if (!emb || emb->shape.size() != 2 || emb->shape[1] != H) Checkpoint::fail("embed_tokens.weight [V][1536] missing");
  const int V = (int)emb->shape[0];
  *gemma = ck.find("per_layer_model_projection.weight_packed") || ck.find("embed_tokens_per_layer.weight");
  if (*gemma) {
    load_gemma(ck, V, ctx);
    return V;
  }
  int NL = 0;
  while (ck.find("layers." + std::to_string(NL) + ".input_layernorm.weight")) ++NL;
  if (NL == 0) Checkpoint::fail("no layers");
  const Tensor* g0 = ck.find("layers.0.mlp.gate_proj.weight_packed");
  if (!g0 || g0->shape.size() != 2) Checkpoint::fail("layers.0.mlp.gate_proj.weight_packed missing");
  const int I = (int)g0->shape[0];
  check(g4v_model_create(G, V, NL, I, ctx), "model_create");
  check(g4v_model_set_embed(G, (const uint16_t*)ck.data(ck.get("embed_tokens.weight", "BF16", (size_t)V * H * 2))),
        "model_set_embed");
  const char* names[7] = {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                          "mlp.gate_proj",    "mlp.up_proj",      "mlp.down_proj"};
  const int Ns[7] = {2048, 256, 256, H, I, I, H}, Ks[7] = {H, H, H, 2048, H, H, I};
  for (int l = 0; l < NL; ++l) {
    const std::string p = "layers." + std::to_string(l) + ".";
    if (!ck.find(p + "self_attn.k_proj.weight_packed"))
      Checkpoint::fail(p + ": no k_proj: a KV-shared layer outside the per-layer-input layout");
    for (int j = 0; j < 7; ++j) set_q4(ck, l, j, p + names[j], Ns[j], Ks[j]);
    const std::vector<float> nv[6] = {
        ck.vec(p + "input_layernorm.weight", H),          ck.vec(p + "post_attention_layernorm.weight", H),
        ck.vec(p + "pre_feedforward_layernorm.weight", H), ck.vec(p + "post_feedforward_layernorm.weight", H),
        ck.vec(p + "self_attn.q_norm.weight", 256),        ck.vec(p + "self_attn.k_norm.weight", 256)};
    const float* nvp[6] = {nv[0].data(), nv[1].data(), nv[2].data(), nv[3].data(), nv[4].data(), nv[5].data()};
    const float scalar = ck.vec(p + "layer_scalar", 1)[0];
    check(g4v_model_set_norms(G, l, nvp, scalar, l % 5 != 4), "model_set_norms");  // E:1225 sliding
  }
  check(g4v_model_set_final_norm(G, ck.vec("norm.weight", H).data()), "model_set_final_norm");
  return V;
}

struct Engine {
  int V = 0, ctx = 4096, pfb = 32, ng_n = 0, ng_len = 3, k_draft = 3;
  // The reference splits attention over its pool's active workers (attn_task, E:1327, 1544): T0 =
  // the ENGINE_CPUS count at start, then set_active(a) (clamped to [1, T0], E:110-112) by every
  // draft step (E:1535: 6, or under ENGINE_ADAPTIVE_THREADS with ENGINE_DRAFT_SAME 8 past the
  // cutoff) and, under ENGINE_ADAPTIVE_THREADS only, by every forward pass (E:1257: 8 when its
  // last position passes the cutoff, else 6).  The count persists between the calls.
  int T0 = 6, active = 6, cut = 192;
  bool adaptive = false, draft_same = true;
  int clamp_active(int a) const { return a < 1 ? T0 : std::min(a, T0); }
  int fwd_splits(int pos0, int M) {  // E:1257 then attn_task's split count
    if (adaptive) active = clamp_active(pos0 + M > cut ? 8 : 6);
    return active;
  }
  int draft_splits(int P) {  // E:1535
    active = clamp_active(draft_same && adaptive && P + 1 > cut ? 8 : 6);
    return active;
  }
  bool drafter = false, stream = false, tree = false, sib_long = false;
  // E:1211 ENGINE_FAKE_CTX: the caches hold fake_n positions of the LCG (E:1249-1250, filled once at
  // start); every request then sits at positions fake_n + ... (E:1599, 1615, 1617) and leaves no
  // reusable prefix (E:1675: kv_len = 0)
  int fake_n = 0;
  float sib_gap = 1.0f;      // E:1629 ENGINE_SIB_GAP: the sibling row is proposed when >= 0
  int pol[3] = {-1, -1, -1};  // E:1513 ENGINE_POLICY: draft count cap per state
  long r1_n = 0, r1_top1 = 0, r1_top2 = 0;  // E:1084, 1659 (over the process)
  long tree_attempts = 0, tree_hits = 0;    // E:1583 (per request), 1648, 1650
  // E:1235 SCR.on (ENGINE_HEAD_SCREEN=1) and the head's screen statistics (E:1245, 1472, 1489;
  // printed at E:1690): rows screened, their survivors, the largest count, and head calls that
  // fell back to the full head.  The library's head always screens; this counts what it reports.
  bool scr_on = false;
  long scr_rows = 0, scr_surv = 0, scr_max = 0, scr_fallback = 0;
  // the stage timers (E:1085 T_LAYERS, T_ATT, T_HEAD, T_DRAFT, N_FWD; E:1672 DECODE_STAGE, E:1691
  // STAGES): forward calls, their wall time less the head's device time, the split-KV attention's
  // and the head's device time from the library's per-class events (g4v_profile, eager launches),
  // and the drafter chains' wall time
  bool stage_prof = false;
  long n_fwd = 0;
  double t_layers = 0, t_att = 0, t_head = 0, t_draft = 0;
  double now() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
  }
  double prof_ms(int a, int b) {  // classes a..b of g4v_profile, ms since it was started
    double ms[G4V_PROF_NTAGS] = {0};
    (void)g4v_profile_read(G, ms, nullptr, nullptr, G4V_PROF_NTAGS);
    double t = 0;
    for (int i = a; i <= b; ++i) t += ms[i];
    return t;
  }
  // one forward call (nf of the reference's fwd calls): N_FWD, T_LAYERS, T_ATT, T_HEAD
  template <class F>
  void fwd_call(int nf, F&& f) {
    const double h0 = stage_prof ? prof_ms(6, 12) : 0.0, a0 = stage_prof ? prof_ms(4, 4) : 0.0;
    const double t = now();
    f();
    const double dt = now() - t;
    n_fwd += nf;
    if (stage_prof) {
      const double dh = (prof_ms(6, 12) - h0) * 1e-3, da = (prof_ms(4, 4) - a0) * 1e-3;
      t_head += dh;
      t_att += da;
      t_layers += std::max(0.0, dt - dh);
    }
  }
  // one head call's rows in evaluation order (row 0, then the lazily evaluated path, E:1475-1488):
  // rows count until the first that overflows the screen, which counts the call's fallback
  void screen_rows(const int* Gr, const int* nsurv, const int* fallback, int n) {
    for (int r = 0; r < n; ++r) {
      if (Gr[r] < 0) continue;
      if (fallback[r]) {
        ++scr_fallback;
        return;
      }
      ++scr_rows;
      scr_surv += nsurv[r];
      scr_max = std::max<long>(scr_max, nsurv[r]);
    }
  }
  void prefill_head() {  // the prefill's head row (E:1472 / 1489 for its head call)
    int ns = 0, fb = 0, g = 0;
    check(g4v_prefill_head_stats(G, &ns, &fb), "prefill_head_stats");
    screen_rows(&g, &ns, &fb, 1);
  }

  // E:1584-1679 for one request
  void run_req(const std::vector<int>& prompt, int nnew, bool print) {
    const int n = (int)prompt.size();
    int start = 0, slot = 0;
    tree_attempts = tree_hits = 0;
    if (fake_n == 0) check(g4v_slot_begin(G, prompt.data(), n, &start, &slot), "slot_begin");
    const int F = fake_n;
    const double t0 = now();
    int g0 = 0;
    std::vector<float> hprev(1536);
    {  // every prompt block is a forward pass (E:1597-1598); only the last block attends split-KV
      const int np = n - start;
      for (int b = 0; b < np; b += pfb) fwd_splits(F + start + b, std::min(pfb, np - b));
    }
    fwd_call((n - start + pfb - 1) / pfb, [&] {  // every block a forward pass (E:1597-1598)
      check(g4v_prefill(G, prompt.data() + start, n - start, F + start, pfb, active, &g0, hprev.data()), "prefill");
    });
    prefill_head();
    const double tp = now() - t0;
    std::vector<int> gen{g0};
    if (print && nnew > 0) {
      printf("FIRST %d\n", g0);
      fflush(stdout);
    }
    if (nnew <= 0) {
      if (F == 0) check(g4v_slot_end(G, prompt.data(), n, nullptr, 0, n - 1), "slot_end");
      if (print) {
        printf("GEN:\nTIMING prompt=%d reused=%d new=%d prefill_s=%.3f decode_tokens=0 decode_s=0 decode_tok_s=0 "
               "tokens_per_round=0 ngram_rounds=0/0 ngram_acc_per_round=0\n",
               n, start, n - start, tp);
        fflush(stdout);
      }
      return;
    }
    const double t1 = now();
    const double layers0 = t_layers, att0 = t_att, head0 = t_head, draft0 = t_draft;  // E:1605
    const long fwd0 = n_fwd;
    size_t emitted = 1;
    auto emit = [&]() {  // E:1612-1614
      if (!stream || !print) return;
      const size_t lim = std::min<size_t>(gen.size(), (size_t)nnew);
      std::string o;
      size_t i = emitted;
      for (; i < lim; ++i) {
        o += ' ' + std::to_string(gen[i]);
        if (is_stop(gen[i])) {
          ++i;
          break;
        }
      }
      if (i > emitted) {
        printf("TOK%s\n", o.c_str());
        fflush(stdout);
        emitted = is_stop(gen[i - 1]) ? lim : i;
      }
    };
    long rounds = 0, ng_rounds = 0, ng_acc = 0;
    int P;
    g4v_verify_result R;
    if (k_draft == 0 || (!drafter && ng_n <= 0)) {  // E:1615: plain decode
      for (int i = 1; i < nnew && !is_stop(gen.back()); ++i) {
        const int t = gen.back();
        fwd_call(1, [&] {
          check(g4v_verify_step(G, &t, 0, 0, F + n + i - 1, fwd_splits(F + n + i - 1, 1), &R, nullptr), "verify_step");
        });
        screen_rows(R.G, R.nsurv, R.fallback, 8);
        gen.push_back(R.commit[0]);
        emit();
      }
      P = F + n + std::max(0, nnew - 1) - 1;
    } else {  // E:1617-1661
      P = F + n - 1;
      int conf = gen.back(), state = 1;
      bool stopped = is_stop(conf), first = true;
      if (ng_n > 0) {  // seq = prompt + generated (E:1625), kept on the device
        std::vector<int> seq(prompt);
        seq.push_back(g0);
        check(g4v_history_set(G, seq.data(), (int)seq.size()), "history_set");
      }
      std::vector<int> app;
      auto commit = [&](int t) {
        gen.push_back(t);
        app.push_back(t);
      };
      while ((int)gen.size() < nnew && !stopped) {
        emit();
        int block[8], nd = 0;
        block[0] = conf;
        int k = std::min(k_draft, 3);
        if (pol[0] >= 0) k = std::min(k, pol[state]);
        if (tree) k = std::min(k, 2);
        bool used_ng = false;
        if (ng_n > 0) {  // E:1624-1628, the round's committed tokens appended first
          check(g4v_prompt_lookup(G, app.data(), (int)app.size(), ng_n, ng_len, block + 1, &nd), "prompt_lookup");
          if (nd > 0) {
            used_ng = true;
            ++ng_rounds;
          }
        }
        app.clear();
        int sec1 = -1;
        float gap1 = -1.0f;
        bool use_sib = false;
        if (!used_ng && drafter && k > 0) {  // E:1632-1645 (TAU 0: every draft is kept)
          int d[3], sec[3];
          float gap[3];
          const double td0 = now();  // E:1646 T_DRAFT
          check(g4v_draft_mtp(G, conf, first ? hprev.data() : nullptr, P, k, draft_splits(P), d, sec, gap, nullptr),
                "draft_mtp");
          t_draft += now() - td0;
          sec1 = sec[0];
          gap1 = gap[0];
          const bool allow_sib = sib_gap >= 0.0f && rounds >= 1 && state < 2 && k >= 2 && sec1 >= 0 && sec1 != d[0];
          const bool sib_cond = (P + 1 + k > ATT_PAR)
                                    ? (sib_long && (gap1 <= 0.85f || (gap1 >= 1.65f && gap1 <= 2.55f)))
                                    : (gap1 <= ((rounds <= 3 || state == 1) ? 2.55f : 1.80f));
          use_sib = allow_sib && sib_cond;  // E:1639-1641: the chain stops after its first draft
          nd = use_sib ? 1 : k;
          for (int j = 0; j < nd; ++j) block[1 + j] = d[j];
        }
        first = false;
        // E:1647-1649
        const int sibling = ((tree || use_sib) && !used_ng && nd >= 1 && sec1 >= 0 && sec1 != block[1]) ? nd + 1 : -1;
        if (sibling >= 0) {
          block[sibling] = sec1;
          ++tree_attempts;
          const bool allow_hit = tree || (P + 1 + sibling <= ATT_PAR && gap1 >= 0.25f);  // E:1650
          fwd_call(1, [&] {
            check(g4v_verify_sibling(G, block, nd, P + 1, fwd_splits(P + 1, nd + 2), allow_hit ? 1 : 0, &R, nullptr),
                  "verify_sibling");
          });
        } else {
          fwd_call(1, [&] {  // E:1649
            check(g4v_verify_step(G, block, nd, 0, P + 1, fwd_splits(P + 1, nd + 1), &R, nullptr), "verify_step");
          });
        }
        screen_rows(R.G, R.nsurv, R.fallback, 8);
        ++rounds;
        if (R.branch == 1) {  // E:1650-1653 the tree hit: row 0's token and the sibling's
          ++tree_hits;
          commit(R.commit[0]);
          if (!is_stop(R.commit[0]) && (int)gen.size() < nnew) commit(R.commit[1]);
          stopped = is_stop(gen.back());
          conf = R.commit[1];
          P += 2;
          state = 1;
          continue;
        }
        if (!used_ng && nd >= 1) {  // E:1655
          ++r1_n;
          if (block[1] == R.G[0]) ++r1_top1;
          else if (sec1 == R.G[0]) ++r1_top2;
        }
        const int nacc = R.nacc;  // E:1656-1660
        if (used_ng) ng_acc += nacc;
        state = nacc == 0 ? 0 : ((!use_sib && nacc == nd) ? 2 : 1);
        for (int i = 0; i <= nacc; ++i) {
          commit(R.commit[i]);
          if (is_stop(R.commit[i])) {
            stopped = true;
            break;
          }
        }
        conf = R.commit[nacc];
        P += nacc + 1;
      }
    }
    emit();
    const double td = now() - t1;
    if (getenv("ENGINE_DECODE_STAGE"))  // E:1672
      fprintf(stderr, "DECODE_STAGE forwards=%ld layers_ms=%.1f split_att_ms=%.1f head_ms=%.1f draft_ms=%.1f total_ms=%.1f\n",
              n_fwd - fwd0, (t_layers - layers0) * 1000, (t_att - att0) * 1000, (t_head - head0) * 1000,
              (t_draft - draft0) * 1000, td * 1000);
    // E:1671: the cache holds the prompt and gen[0 .. P - n] (E:1675: nothing reusable past a fake context)
    if (F == 0) check(g4v_slot_end(G, prompt.data(), n, gen.data(), (int)gen.size(), P), "slot_end");
    if ((int)gen.size() > nnew) gen.resize(nnew);
    for (size_t i = 0; i < gen.size(); ++i)
      if (is_stop(gen[i])) {
        gen.resize(i + 1);
        break;
      }
    if (print) {
      fprintf(stderr, "RANK1 rounds=%ld top1=%ld top2_only=%ld TREE attempts=%ld hits=%ld\n", r1_n, r1_top1, r1_top2,
              tree_attempts, tree_hits);  // E:1673
      fflush(stderr);
      printf("GEN:");
      for (int g : gen) printf(" %d", g);
      printf("\n");
      const int produced = std::max(0, (int)gen.size() - 1);
      printf("TIMING prompt=%d reused=%d new=%d prefill_s=%.3f decode_tokens=%d decode_s=%.3f decode_tok_s=%.2f "
             "tokens_per_round=%.2f ngram_rounds=%ld/%ld ngram_acc_per_round=%.2f slot=%d\n",
             n, start, n - start, tp, produced, td, produced / td, rounds ? (double)produced / rounds : 1.0,
             ng_rounds, rounds, ng_rounds ? (double)ng_acc / ng_rounds : 0.0, slot);
      fflush(stdout);
    }
  }
};

}  // namespace

int main(int argc, char** argv) {
  if (argc < 5) {
    fprintf(stderr, "usage: %s <checkpoint dir | synth:SEED:V:NL:I> <index> <prompt.ids | -> <nnew>\n", argv[0]);
    return 2;
  }
  unsigned long long seed = 0;
  int V = 0, NL = 0, I = 0;
  const bool synth = sscanf(argv[1], "synth:%llu:%d:%d:%d", &seed, &V, &NL, &I) == 4;
  Engine e;
  e.V = V;
  e.ctx = env_int("ENGINE_CTX", 4096);
  e.pfb = env_int("ENGINE_PREFILL_BLOCK", 32);
  e.ng_n = env_int("ENGINE_NGRAM", 0);
  e.ng_len = std::min(7, env_int("ENGINE_NGLEN", 3));  // E:1514
  e.k_draft = env_int("ENGINE_K", 3);
  e.stream = getenv("ENGINE_STREAM") != nullptr;
  e.tree = env_int("ENGINE_TREE", 0) == 1;
  e.sib_long = getenv("ENGINE_SIB_LONG") != nullptr;
  if (const char* g = getenv("ENGINE_SIB_GAP")) e.sib_gap = (float)atof(g);
  if (const char* pp = getenv("ENGINE_POLICY")) sscanf(pp, "%d,%d,%d", &e.pol[0], &e.pol[1], &e.pol[2]);
  {  // the pool size (E:75-77, E:1215): one split per active worker
    int ncpu = 6;
    if (const char* c = getenv("ENGINE_CPUS")) {
      ncpu = 1;
      for (const char* p = c; *p; ++p) ncpu += *p == ',';
    }
    e.T0 = e.active = std::max(1, std::min(16, ncpu));
    e.adaptive = getenv("ENGINE_ADAPTIVE_THREADS") != nullptr;
    e.cut = env_int("ENGINE_THREAD_CUTOFF", 192);  // E:1257 (default ATT_PAR), E:1533
    e.draft_same = !(getenv("ENGINE_DRAFT_SAME") && atoi(getenv("ENGINE_DRAFT_SAME")) == 0);  // E:1532
  }
  // E:1210 G_I8 and E:1600 DEC_I8: the prompt's linear layers run W4A8 when ENGINE_PREFILL_INT8=1,
  // and then the decode's verify passes of two rows or more too unless ENGINE_DECODE_INT8=0
  // (g4v_set_decode_int8)
  // settings whose reference paths this engine does not restate end the process (exit code 2)
  // rather than run another path silently: the split-KV threshold and switch (E:1212-1214), the
  // attn_tile switch ENGINE_NO_TILED (E:1213, 1328: run_mh for blocks attn_tile takes), and the
  // draft chain's probability cut ENGINE_TAU > 0 (E:1515, 1561, 1644); a fake context with more
  // than one cache slot (E:1573-1593 would park and swap the fake rows)
  if (env_int("ENGINE_ATT_PAR", ATT_PAR) != ATT_PAR || env_int("ENGINE_SPLITKV", 1) == 0 ||
      getenv("ENGINE_NO_TILED") || (getenv("ENGINE_TAU") && atof(getenv("ENGINE_TAU")) > 0.0)) {
    fprintf(stderr, "g4v_engine: ENGINE_ATT_PAR other than %d, ENGINE_SPLITKV=0, ENGINE_NO_TILED and ENGINE_TAU > 0 "
                    "are not supported (E:1212-1214, 1515)\n", ATT_PAR);
    return 2;
  }
  e.fake_n = env_int("ENGINE_FAKE_CTX", 0);
  if (e.fake_n < 0 || e.fake_n >= e.ctx || (e.fake_n > 0 && env_int("ENGINE_SLOTS", 1) > 1)) {
    fprintf(stderr, "g4v_engine: ENGINE_FAKE_CTX needs 0 <= n < ENGINE_CTX and one cache slot (E:1211, 1573)\n");
    return 2;
  }
  const bool samepos = env_int("ENGINE_DRAFT_SAMEPOS", 0) == 1;  // E:1516
  const bool g_i8 = env_int("ENGINE_PREFILL_INT8", 0) == 1;
  const bool dec_i8 = !(getenv("ENGINE_DECODE_INT8") && atoi(getenv("ENGINE_DECODE_INT8")) == 0);
  check(g4v_create(0, &G), "create");
  e.scr_on = getenv("ENGINE_HEAD_SCREEN") && atoi(getenv("ENGINE_HEAD_SCREEN")) == 1;  // E:1235
  e.stage_prof = getenv("ENGINE_DECODE_STAGE") || getenv("ENGINE_STAGE_PROF");
  if (e.stage_prof) {  // per-class events on eagerly launched passes (a replayed graph records none)
    check(g4v_set_graphs(G, 0), "set_graphs");
    check(g4v_profile(G, (1u << G4V_PROF_NTAGS) - 1), "profile");
  }
  check(g4v_set_prefill_int8(G, g_i8 ? 1 : 0), "set_prefill_int8");
  Checkpoint ck;
  bool gemma = false;
  if (synth) {
    check(g4v_model_synth(G, seed, V, NL, I, e.ctx), "model_synth");
  } else {
    ck.open_files(argv[1], argv[2]);
    V = load_checkpoint(ck, e.ctx, &gemma);
    e.V = V;
    NL = 0;
    while (ck.find("layers." + std::to_string(NL) + ".input_layernorm.weight")) ++NL;
  }
  if (g_i8 && dec_i8) check(g4v_set_decode_int8(G, 1), "set_decode_int8");
  const char* dseed = getenv("ENGINE_DRAFTER_SEED");
  Checkpoint dk;
  if (gemma && e.k_draft > 0) {  // E:1519-1528: the drafter checkpoint main() loads when ENGINE_K > 0
    const char* dc = getenv("ENGINE_DRAFTER_DIR") ? getenv("ENGINE_DRAFTER_DIR") : "ckpt-e2b-assistant";
    const char* di = getenv("ENGINE_DRAFTER_INDEX") ? getenv("ENGINE_DRAFTER_INDEX") : "runs/drafter_index.tsv";
    dk.open_files(dc, di);
    load_drafter(dk);
    e.drafter = true;
  }
  if (!gemma && e.k_draft > 0 && NL >= 15 && V % 2048 == 0 && (synth || dseed)) {
    check(g4v_drafter_synth(G, dseed ? strtoull(dseed, nullptr, 10) : seed + 1), "drafter_synth");
    e.drafter = true;
  }
  check(g4v_slots_init(G, std::max(1, env_int("ENGINE_SLOTS", 1)), env_int("ENGINE_SLOT_MIN_REUSE", 32)), "slots_init");
  if (samepos) check(g4v_set_draft_samepos(G, 1), "set_draft_samepos");
  if (e.fake_n > 0) check(g4v_model_fake_ctx(G, e.fake_n, 12345), "model_fake_ctx");  // E:1249-1250, before the warm-up
  {  // E:1578: one warm-up pass at position 0 (the cache is not marked valid by it)
    const int w = 2;
    int g = 0;
    e.fwd_call(1, [&] { check(g4v_prefill(G, &w, 1, 0, e.pfb, e.fwd_splits(0, 1), &g, nullptr), "warm-up"); });
    e.prefill_head();
  }
  if (getenv("ENGINE_SERVE")) {
    std::string line;
    while (std::getline(std::cin, line)) {
      if (line.rfind("BENCH_MODE ", 0) == 0) {  // E:1683
        std::stringstream ms(line);
        std::string cmd;
        int k = -1, tree = -1;
        ms >> cmd >> k >> tree;
        if (k >= 1 && k <= 3 && tree >= 0 && tree <= 1 && e.drafter) {
          e.k_draft = k;
          e.tree = tree == 1;
          printf("MODE k=%d tree=%d\n", k, tree);
        } else {
          printf("MODE_ERROR\n");
        }
        fflush(stdout);
        continue;
      }
      std::stringstream ss(line);
      int nn;
      if (!(ss >> nn)) continue;
      std::vector<int> pr;
      std::string w;
      while (ss >> w) pr.push_back(atoi(w.c_str()));
      if (pr.empty()) continue;
      e.run_req(pr, nn, true);
    }
  } else {
    std::vector<int> prompt;
    std::ifstream f(argv[3]);
    int v;
    while (f >> v) prompt.push_back(v);
    if (prompt.empty()) {
      fprintf(stderr, "empty prompt %s\n", argv[3]);
      return 2;
    }
    e.run_req(prompt, atoi(argv[4]), true);
    if (e.scr_on && e.scr_rows)  // E:1690
      fprintf(stderr, "SCREEN rows=%ld survivors mean=%.1f max=%ld fallbacks=%ld\n", e.scr_rows,
              (double)e.scr_surv / e.scr_rows, e.scr_max, e.scr_fallback);
  }
  if (getenv("ENGINE_STAGE_PROF"))  // E:1691
    fprintf(stderr, "STAGES total over %ld fwd calls (ms): layers %.0f (of which split-KV attention %.0f) | head %.0f | "
                    "drafter %.0f\n", e.n_fwd, e.t_layers * 1e3, e.t_att * 1e3, e.t_head * 1e3, e.t_draft * 1e3);
  fflush(stderr);
  fflush(stdout);
  g4v_destroy(G);
  return 0;
}
