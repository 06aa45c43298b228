// ref_engine_screen.cpp -- runs the reference engine's own main() and writes out the head
// screen it builds.
//
// TEST INFRASTRUCTURE.  Built by oracle/Makefile from the reference sources where they lie
// (the engine is included with `#define main engine_main`, the trick the reference's
// bench/attn_bench.cpp:2-4 uses); the output goes to oracle/_ref/ only.
//
// The screen build is a lambda inside main() (E:1235-1244 of engine/gemma4_engine.cpp), so
// no call reaches it from outside.  This program runs main() itself, unchanged, on a
// checkpoint directory (model.safetensors + the tensor index TSV, E:1214-1216) with
// ENGINE_HEAD_SCREEN=1, in a thread whose stderr is a pipe read here.  main() prints
// "head screen built" (E:1245) once the build's worker pool has finished; the program then
// copies the global screen (SCR.w [262144][768] u8, SCR.s [262144][48] bf16, SCR.coef
// [262144] f32) to the output file in that order and ends the process.  main() runs with
// ENGINE_SERVE set, ENGINE_K=0 (no drafter) and its stdin on a pipe nothing is ever written to, so after its warm-up
// pass it waits in its request loop (E:1673) instead of reaching its _exit (E:1698) while the
// screen is being copied.
//
// usage: ref_engine_screen <ckpt dir> <index.tsv> <prompt file> <out.bin>
#include <thread>
#define main engine_main
#include G4_REF_ENGINE
#undef main
#include <unistd.h>

int main(int argc, char** argv) {
  if (argc != 5) {
    fprintf(stderr, "usage: %s <ckpt dir> <index.tsv> <prompt file> <out.bin>\n", argv[0]);
    return 2;
  }
  int fds[2], in_fds[2];
  if (pipe(fds) != 0 || pipe(in_fds) != 0) return 3;
  const int err_fd = dup(2);
  dup2(fds[1], 2);     // the engine's stderr goes to the pipe
  dup2(in_fds[0], 0);  // its stdin: a pipe whose write end stays open and silent
  setenv("ENGINE_HEAD_SCREEN", "1", 1);
  setenv("ENGINE_SERVE", "1", 1);
  setenv("ENGINE_K", "0", 1);  // no drafter checkpoint (E:1517-1519)
  static char* av[5] = {argv[0], argv[1], argv[2], argv[3], (char*)"0"};
  std::thread([] { engine_main(5, av); }).detach();
  FILE* in = fdopen(fds[0], "r");
  char line[4096];
  bool built = false;
  while (fgets(line, sizeof line, in)) {
    if (write(err_fd, line, strlen(line)) < 0) break;
    if (strstr(line, "head screen built")) {
      built = true;
      break;
    }
  }
  if (!built) {
    dprintf(err_fd, "ref_engine_screen: the engine ended before building the screen\n");
    _exit(4);
  }
  FILE* o = fopen(argv[4], "wb");
  if (!o) _exit(5);
  const bool ok = fwrite(SCR.w.data(), 1, SCR.w.size(), o) == SCR.w.size() &&
                  fwrite(SCR.s.data(), 2, SCR.s.size(), o) == SCR.s.size() &&
                  fwrite(SCR.coef.data(), 4, SCR.coef.size(), o) == SCR.coef.size();
  fclose(o);
  dprintf(err_fd, "ref_engine_screen: wrote %zu + %zu + %zu bytes\n", SCR.w.size(), SCR.s.size() * 2,
          SCR.coef.size() * 4);
  _exit(ok ? 0 : 6);
}
