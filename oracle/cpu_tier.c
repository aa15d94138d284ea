/*
 * cpu_tier.c — TEST INFRASTRUCTURE ONLY: the reference's *timed* CPU tier,
 * used by bench.py's cpu_baseline leg (never by the shipped library, never as
 * a parity oracle: its f32 accumulation differs from the scalar tier).
 *
 * Restates what the reference runs at decode time on an x86_64 host:
 *   - the runtime-selected SIMD dots (simd_x86.rs:18-29): AVX-VNNI for Q8 and
 *     Q4_0 when the CPU has avx_vnni (97-156), else AVX2+FMA (163-244); AVX2
 *     for Q4_K (252-299) and the dense f32 dot (52-72); Q6_K stays scalar
 *     (kquant.rs:361);
 *   - the persistent spin-then-park work-stealing pool (pool.rs:95-307):
 *     N-1 workers spawned once, a job of chunk indices claimed from a shared
 *     counter by the workers and the submitter, the submitter returning when
 *     every chunk is done;
 *   - run_rows / run_rows_multi chunking (matmul.rs:192-232, 318-350):
 *     serial below 2^18 (decode) / 2^20 (batched) MACs, else chunks of
 *     max(ceil(rows / (4 * threads)), 16) rows (4 for batched);
 *   - default_threads = min(nproc, 8) (threading.rs:46-53), overridable.
 */
#define _GNU_SOURCE
#include <immintrin.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "prana_oracle.h"

/* ------------------------------------------------------------------ SIMD dots */
__attribute__((target("avx2"))) static float hsum8(__m256 v) {
  __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
  s = _mm_add_ps(s, _mm_movehl_ps(s, s));
  s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
  return _mm_cvtss_f32(s);
}

/* x.y of 32 signed bytes as 8 i32 lanes: |x| times y with x's sign moved
 * onto it, u8 x i8 pairs to i16, i16 pairs to i32 (simd_x86.rs:82-88). */
__attribute__((target("avx2"))) static __m256i i8_dot8(__m256i x, __m256i y) {
  const __m256i ax = _mm256_sign_epi8(x, x), sy = _mm256_sign_epi8(y, x);
  return _mm256_madd_epi16(_mm256_maddubs_epi16(ax, sy), _mm256_set1_epi16(1));
}

__attribute__((target("avx2,fma"))) static float t_dot_f32(const float *a, const float *b, size_t n) {
  __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
  const size_t chunks = n / 16;
  for (size_t i = 0; i < chunks; i++) {
    acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + 16 * i), _mm256_loadu_ps(b + 16 * i), acc0);
    acc1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + 16 * i + 8), _mm256_loadu_ps(b + 16 * i + 8), acc1);
  }
  float sum = hsum8(_mm256_add_ps(acc0, acc1));
  for (size_t i = chunks * 16; i < n; i++) sum += a[i] * b[i];
  return sum;
}

__attribute__((target("avx2,fma"))) static float t_dot_q8(const int8_t *qa, const float *sa, const int8_t *qw,
                                                          const float *sw, size_t groups) {
  __m256 acc = _mm256_setzero_ps();
  for (size_t g = 0; g < groups; g++) {
    const __m256i a = _mm256_loadu_si256((const __m256i *)(qa + 32 * g));
    const __m256i w = _mm256_loadu_si256((const __m256i *)(qw + 32 * g));
    acc = _mm256_fmadd_ps(_mm256_cvtepi32_ps(i8_dot8(w, a)), _mm256_set1_ps(sw[g] * sa[g]), acc);
  }
  return hsum8(acc);
}

__attribute__((target("avx2,fma,avxvnni"))) static float t_dot_q8_vnni(const int8_t *qa, const float *sa,
                                                                       const int8_t *qw, const float *sw,
                                                                       size_t groups) {
  __m256 acc = _mm256_setzero_ps();
  for (size_t g = 0; g < groups; g++) {
    const __m256i a = _mm256_loadu_si256((const __m256i *)(qa + 32 * g));
    const __m256i w = _mm256_loadu_si256((const __m256i *)(qw + 32 * g));
    const __m256i p = _mm256_dpbusd_avx_epi32(_mm256_setzero_si256(), _mm256_sign_epi8(w, w), _mm256_sign_epi8(a, w));
    acc = _mm256_fmadd_ps(_mm256_cvtepi32_ps(p), _mm256_set1_ps(sw[g] * sa[g]), acc);
  }
  return hsum8(acc);
}

/* 16 Q4_0 quant bytes -> 32 centred bytes q - 8 (elements 0..15 low nibbles,
 * 16..31 high nibbles; simd_x86.rs:189-199). */
__attribute__((target("avx2"))) static __m256i q40_i8(const uint8_t *qs) {
  const __m128i b = _mm_loadu_si128((const __m128i *)qs), m = _mm_set1_epi8(0x0F);
  const __m128i lo = _mm_and_si128(b, m), hi = _mm_and_si128(_mm_srli_epi16(b, 4), m);
  return _mm256_sub_epi8(_mm256_set_m128i(hi, lo), _mm256_set1_epi8(8));
}

/* Two blocks per step on independent accumulators (simd_x86.rs:210-244). */
__attribute__((target("avx2,fma"))) static float t_dot_q40(const int8_t *qa, const float *sa, const uint8_t *row,
                                                           const float *ds, size_t nb) {
  __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
  size_t i = 0;
  for (; i + 2 <= nb; i += 2) {
    const __m256i w0 = q40_i8(row + i * 18 + 2), w1 = q40_i8(row + (i + 1) * 18 + 2);
    const __m256i a0 = _mm256_loadu_si256((const __m256i *)(qa + 32 * i));
    const __m256i a1 = _mm256_loadu_si256((const __m256i *)(qa + 32 * i + 32));
    acc0 = _mm256_fmadd_ps(_mm256_cvtepi32_ps(i8_dot8(w0, a0)), _mm256_set1_ps(ds[i] * sa[i]), acc0);
    acc1 = _mm256_fmadd_ps(_mm256_cvtepi32_ps(i8_dot8(w1, a1)), _mm256_set1_ps(ds[i + 1] * sa[i + 1]), acc1);
  }
  if (i < nb) {
    const __m256i w = q40_i8(row + i * 18 + 2);
    const __m256i a = _mm256_loadu_si256((const __m256i *)(qa + 32 * i));
    acc0 = _mm256_fmadd_ps(_mm256_cvtepi32_ps(i8_dot8(w, a)), _mm256_set1_ps(ds[i] * sa[i]), acc0);
  }
  return hsum8(_mm256_add_ps(acc0, acc1));
}

__attribute__((target("avx2,fma,avxvnni"))) static float t_dot_q40_vnni(const int8_t *qa, const float *sa,
                                                                        const uint8_t *row, const float *ds,
                                                                        size_t nb) {
  const __m256i z = _mm256_setzero_si256();
  __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
  size_t i = 0;
  for (; i + 2 <= nb; i += 2) {
    const __m256i w0 = q40_i8(row + i * 18 + 2), w1 = q40_i8(row + (i + 1) * 18 + 2);
    const __m256i a0 = _mm256_loadu_si256((const __m256i *)(qa + 32 * i));
    const __m256i a1 = _mm256_loadu_si256((const __m256i *)(qa + 32 * i + 32));
    const __m256i p0 = _mm256_dpbusd_avx_epi32(z, _mm256_sign_epi8(w0, w0), _mm256_sign_epi8(a0, w0));
    const __m256i p1 = _mm256_dpbusd_avx_epi32(z, _mm256_sign_epi8(w1, w1), _mm256_sign_epi8(a1, w1));
    acc0 = _mm256_fmadd_ps(_mm256_cvtepi32_ps(p0), _mm256_set1_ps(ds[i] * sa[i]), acc0);
    acc1 = _mm256_fmadd_ps(_mm256_cvtepi32_ps(p1), _mm256_set1_ps(ds[i + 1] * sa[i + 1]), acc1);
  }
  if (i < nb) {
    const __m256i w = q40_i8(row + i * 18 + 2);
    const __m256i a = _mm256_loadu_si256((const __m256i *)(qa + 32 * i));
    const __m256i p = _mm256_dpbusd_avx_epi32(z, _mm256_sign_epi8(w, w), _mm256_sign_epi8(a, w));
    acc0 = _mm256_fmadd_ps(_mm256_cvtepi32_ps(p), _mm256_set1_ps(ds[i] * sa[i]), acc0);
  }
  return hsum8(_mm256_add_ps(acc0, acc1));
}

/* Q4_K: per 32-group the integer dot as an exact horizontal sum, then the
 * scalar tier's f32 term (simd_x86.rs:252-299; equal to the scalar tier bit
 * for bit, the group sums being exact in f32). */
__attribute__((target("avx2,fma"))) static float t_dot_q4k(const int8_t *qa, const float *sa, const int32_t *suma,
                                                           const uint8_t *row, const float *ds, size_t nb) {
  const __m256i mask = _mm256_set1_epi8(0x0F), ones = _mm256_set1_epi16(1);
  float total = 0.0f;
  for (size_t b = 0; b < nb; b++) {
    const uint8_t *blk = row + b * 144;
    const float d = ds[2 * b], dmin = ds[2 * b + 1];
    const int8_t *pa = qa + 256 * b;
    for (int pair = 0; pair < 4; pair++) {
      const __m256i bytes = _mm256_loadu_si256((const __m256i *)(blk + 16 + 32 * pair));
      const __m256i lo = _mm256_and_si256(bytes, mask), hi = _mm256_and_si256(_mm256_srli_epi16(bytes, 4), mask);
      const __m256i a_lo = _mm256_loadu_si256((const __m256i *)(pa + 64 * pair));
      const __m256i a_hi = _mm256_loadu_si256((const __m256i *)(pa + 64 * pair + 32));
      const float s1 = hsum8(_mm256_cvtepi32_ps(_mm256_madd_epi16(_mm256_maddubs_epi16(lo, a_lo), ones)));
      const float s2 = hsum8(_mm256_cvtepi32_ps(_mm256_madd_epi16(_mm256_maddubs_epi16(hi, a_hi), ones)));
      const size_t g_lo = 8 * b + 2 * pair, g_hi = g_lo + 1;
      float sc1, m1, sc2, m2;
      po_q4k_scale_min(2 * pair, blk + 4, &sc1, &m1);
      po_q4k_scale_min(2 * pair + 1, blk + 4, &sc2, &m2);
      total += sa[g_lo] * (d * sc1 * s1 - dmin * m1 * (float)suma[g_lo]);
      total += sa[g_hi] * (d * sc2 * s2 - dmin * m2 * (float)suma[g_hi]);
    }
  }
  return total;
}

static int g_has_avx2 = -1, g_has_vnni = -1;
static void detect(void) {
  if (g_has_avx2 >= 0) return;
  __builtin_cpu_init();
  g_has_avx2 = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
  g_has_vnni = g_has_avx2 && __builtin_cpu_supports("avxvnni");
}

/* The tier's row dot for one of the oracle's formats (kind as in
 * po_mat_kind: 0 F32, 1 Q8, 2 Q4_0, 3 Q4_K, 4 Q6_K). */
float pt_row_dot(int kind, const float *x, const float *w, const int8_t *qa, const float *sa, const int32_t *suma,
                 const int8_t *qw, const float *sw, const uint8_t *row, const float *ds, size_t k) {
  detect();
  switch (kind) {
    case 0: return g_has_avx2 ? t_dot_f32(x, w, k) : po_dot_f32(x, w, k);
    case 1:
      if (g_has_vnni) return t_dot_q8_vnni(qa, sa, qw, sw, k / 32);
      return g_has_avx2 ? t_dot_q8(qa, sa, qw, sw, k / 32) : po_dot_q8_q8(qa, sa, qw, sw, k / 32);
    case 2:
      if (g_has_vnni) return t_dot_q40_vnni(qa, sa, row, ds, k / 32);
      return g_has_avx2 ? t_dot_q40(qa, sa, row, ds, k / 32) : po_dot_q40_q8(qa, sa, suma, row, ds, k / 32);
    case 3: return g_has_avx2 ? t_dot_q4k(qa, sa, suma, row, ds, k / 256) : po_dot_q4k_q8(qa, sa, suma, row, ds, k / 256);
    default: return po_dot_q6k_q8(qa, sa, suma, row, ds, k / 256);
  }
}

const char *pt_simd_tier(void) {
  detect();
  if (g_has_vnni) return "avx_vnni (Q8, Q4_0), avx2+fma (Q4_K, f32), scalar (Q6_K)";
  if (g_has_avx2) return "avx2+fma (Q8, Q4_0, Q4_K, f32), scalar (Q6_K)";
  return "scalar";
}

/* ------------------------------------------------------------------ pool */
enum { kSpinIters = 200000, kMaxWorkers = 255 };

typedef struct {
  void (*fn)(void *ctx, size_t chunk);
  void *ctx;
  uint32_t n_chunks;
  atomic_uint next, remaining, users;
} pool_job;

static struct {
  int threads;  /* workers spawned + the submitter */
  int active;   /* threads that take part in jobs (<= threads) */
  atomic_ullong epoch;
  pthread_mutex_t slot_mu;
  pthread_cond_t work_cv;
  pool_job *slot;
  atomic_uint parked;
  pthread_mutex_t done_mu;
  pthread_cond_t done_cv;
  atomic_int submitter_waiting;
  pthread_mutex_t submit_mu;
} P = {0, 0, 0, PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER, NULL, 0, PTHREAD_MUTEX_INITIALIZER,
       PTHREAD_COND_INITIALIZER, 0, PTHREAD_MUTEX_INITIALIZER};

static void run_chunks(pool_job *j) {
  for (;;) {
    const uint32_t i = atomic_fetch_add_explicit(&j->next, 1, memory_order_relaxed);
    if (i >= j->n_chunks) break;
    j->fn(j->ctx, i);
    atomic_fetch_sub_explicit(&j->remaining, 1, memory_order_acq_rel);
  }
}

static void *worker(void *arg) {
  const int index = (int)(intptr_t)arg;  /* 1..threads-1; the submitter is 0 */
  unsigned long long seen = 0;
  for (;;) {
    unsigned spins = 0;
    for (;;) {  /* wait for a new epoch: spin, then park */
      const unsigned long long e = atomic_load_explicit(&P.epoch, memory_order_acquire);
      if (e != seen) {
        seen = e;
        break;
      }
      if (spins < kSpinIters) {
        spins++;
        _mm_pause();
      } else {
        pthread_mutex_lock(&P.slot_mu);
        atomic_fetch_add(&P.parked, 1);
        if (atomic_load_explicit(&P.epoch, memory_order_acquire) == seen) pthread_cond_wait(&P.work_cv, &P.slot_mu);
        atomic_fetch_sub(&P.parked, 1);
        pthread_mutex_unlock(&P.slot_mu);
        spins = 0;
      }
    }
    if (index >= P.active) continue;  /* not part of the current team size */
    pthread_mutex_lock(&P.slot_mu);  /* take a reference to the published job */
    pool_job *j = P.slot;
    if (j) atomic_fetch_add(&j->users, 1);
    pthread_mutex_unlock(&P.slot_mu);
    if (!j) continue;
    run_chunks(j);
    const int last = atomic_load_explicit(&j->remaining, memory_order_acquire) == 0;
    atomic_fetch_sub(&j->users, 1);
    if (last && atomic_load(&P.submitter_waiting)) {
      pthread_mutex_lock(&P.done_mu);
      pthread_cond_broadcast(&P.done_cv);
      pthread_mutex_unlock(&P.done_mu);
    }
  }
  return NULL;
}

static int default_threads(void) {
  const char *e = getenv("PRANA_THREADS");
  if (e && atoi(e) > 0) return atoi(e);
  const long n = sysconf(_SC_NPROCESSORS_ONLN);
  return n < 1 ? 1 : (n > 8 ? 8 : (int)n);
}

/* Size the pool (threads <= 0: the reference default): workers are spawned
 * once and kept; asking for fewer threads later leaves the extra workers
 * waiting outside the jobs. Call between jobs, from the submitting thread. */
int pt_pool_start(int threads) {
  int want = threads > 0 ? threads : default_threads();
  if (want > kMaxWorkers + 1) want = kMaxWorkers + 1;
  for (int i = P.threads > 0 ? P.threads : 1; i < want; i++) {
    pthread_t t;
    pthread_create(&t, NULL, worker, (void *)(intptr_t)i);
    pthread_detach(t);
  }
  if (want > P.threads) P.threads = want;
  P.active = want;
  return P.active;
}

/* Run fn(ctx, c) for c in 0..n_chunks over the pool and the caller. */
void pt_pool_run(size_t n_chunks, void (*fn)(void *, size_t), void *ctx) {
  if (n_chunks == 0) return;
  if (n_chunks == 1 || P.active <= 1) {
    for (size_t c = 0; c < n_chunks; c++) fn(ctx, c);
    return;
  }
  pthread_mutex_lock(&P.submit_mu);
  pool_job j;
  j.fn = fn;
  j.ctx = ctx;
  j.n_chunks = (uint32_t)n_chunks;
  atomic_init(&j.next, 0);
  atomic_init(&j.remaining, (unsigned)n_chunks);
  atomic_init(&j.users, 0);
  pthread_mutex_lock(&P.slot_mu);
  P.slot = &j;
  atomic_fetch_add_explicit(&P.epoch, 1, memory_order_release);
  pthread_mutex_unlock(&P.slot_mu);
  if (atomic_load_explicit(&P.parked, memory_order_acquire) > 0) {
    pthread_mutex_lock(&P.slot_mu);
    pthread_cond_broadcast(&P.work_cv);
    pthread_mutex_unlock(&P.slot_mu);
  }
  run_chunks(&j);
  unsigned spins = 0;
  while (atomic_load_explicit(&j.remaining, memory_order_acquire) != 0) {
    if (spins < kSpinIters) {
      spins++;
      _mm_pause();
    } else {
      pthread_mutex_lock(&P.done_mu);
      atomic_store(&P.submitter_waiting, 1);
      if (atomic_load_explicit(&j.remaining, memory_order_acquire) != 0) {
        struct timespec ts;
        clock_gettime(CLOCK_REALTIME, &ts);
        ts.tv_nsec += 1000000;  /* 1 ms bounds a lost wake-up */
        if (ts.tv_nsec >= 1000000000) {
          ts.tv_sec++;
          ts.tv_nsec -= 1000000000;
        }
        pthread_cond_timedwait(&P.done_cv, &P.done_mu, &ts);
      }
      atomic_store(&P.submitter_waiting, 0);
      pthread_mutex_unlock(&P.done_mu);
    }
  }
  pthread_mutex_lock(&P.slot_mu);  /* no new worker can take the job now */
  P.slot = NULL;
  pthread_mutex_unlock(&P.slot_mu);
  while (atomic_load_explicit(&j.users, memory_order_acquire) != 0) _mm_pause();
  pthread_mutex_unlock(&P.submit_mu);
}

int pt_pool_threads(void) { return P.active; }
