/* host_stream.c -- host read bandwidth (TEST INFRASTRUCTURE: the CPU-baseline leg of bench.py
 * reports it beside the reference's timing on the same host).
 *
 * The method of the reference's bench/stream_bw.cpp:10-19: one buffer larger than the last-level
 * cache, split into contiguous per-thread slices, each thread pinned to one CPU and summing its
 * slice with wide loads for a number of passes; bandwidth = passes x bytes / wall time.  Written
 * here in plain C (the compiler vectorises the 8-lane float sums at -O3 -march=x86-64-v3). */
#define _GNU_SOURCE
#include <pthread.h>
#include <sched.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

typedef struct {
  const float* p;
  size_t n;  /* floats */
  int cpu, passes;
  float out[8];
} hs_job;

static void* hs_work(void* arg) {
  hs_job* j = (hs_job*)arg;
  cpu_set_t s;
  CPU_ZERO(&s);
  CPU_SET(j->cpu, &s);
  pthread_setaffinity_np(pthread_self(), sizeof s, &s);
  float acc[8] = {0};
  for (int r = 0; r < j->passes; ++r)
    for (size_t i = 0; i + 8 <= j->n; i += 8)
      for (int k = 0; k < 8; ++k) acc[k] += j->p[i + k];
  memcpy(j->out, acc, sizeof acc);
  return NULL;
}

/* GB/s of `passes` reads of a `bytes` buffer by n threads pinned to cpus[0..n-1]; < 0 on error */
double g4h_read_gbs(const int* cpus, int n, size_t bytes, int passes) {
  if (n < 1 || n > 256 || passes < 1) return -1.0;
  bytes = bytes / (64 * (size_t)n) * 64 * (size_t)n;
  float* buf = (float*)aligned_alloc(64, bytes);
  if (!buf) return -1.0;
  memset(buf, 1, bytes);
  hs_job* jobs = (hs_job*)calloc((size_t)n, sizeof(hs_job));
  pthread_t* th = (pthread_t*)calloc((size_t)n, sizeof(pthread_t));
  const size_t per = bytes / sizeof(float) / (size_t)n;
  for (int t = 0; t < n; ++t) {
    jobs[t].p = buf + per * (size_t)t;
    jobs[t].n = per;
    jobs[t].cpu = cpus[t];
    jobs[t].passes = passes;
  }
  struct timespec a, b;
  clock_gettime(CLOCK_MONOTONIC, &a);
  for (int t = 0; t < n; ++t) pthread_create(&th[t], NULL, hs_work, &jobs[t]);
  for (int t = 0; t < n; ++t) pthread_join(th[t], NULL);
  clock_gettime(CLOCK_MONOTONIC, &b);
  const double s = (double)(b.tv_sec - a.tv_sec) + 1e-9 * (double)(b.tv_nsec - a.tv_nsec);
  volatile float sink = 0;
  for (int t = 0; t < n; ++t) sink += jobs[t].out[0];
  (void)sink;
  free(th);
  free(jobs);
  free(buf);
  return (double)passes * (double)bytes / s / 1e9;
}
