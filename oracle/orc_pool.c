/*
 * orc_pool.c -- the oracle's persistent worker pool. TEST INFRASTRUCTURE.
 *
 * Restates app::Pool (runtime/include/runtime/pool.hpp:18-39,
 * runtime/src/pool.cpp:28-110): N persistent workers, a generation counter and
 * a CUMULATIVE completion count (a count-down released waiters early in the
 * reference's history, pool.cpp:62-81). run(f) calls f(w, nw) once on every
 * worker, worker 0 being the caller, and returns when all have finished.
 */
#include "orc_internal.h"

#include <pthread.h>
#include <stdlib.h>
#include <unistd.h>

typedef struct {
  int n;
  pthread_t *thr;
  pthread_mutex_t mu;
  pthread_cond_t cv_work, cv_done;
  orc_task_fn fn;
  void *arg;
  long gen;
  long completed;
  int quit;
} orc_pool_t;

static orc_pool_t g_pool;
static int g_pool_up = 0;
static pthread_mutex_t g_pool_init_mu = PTHREAD_MUTEX_INITIALIZER;

typedef struct { int w; } worker_arg;

static void *worker_main(void *p) {
  const int w = ((worker_arg *)p)->w;
  free(p);
  long seen = 0;
  for (;;) {
    pthread_mutex_lock(&g_pool.mu);
    while (!g_pool.quit && g_pool.gen == seen)
      pthread_cond_wait(&g_pool.cv_work, &g_pool.mu);
    if (g_pool.quit) {
      pthread_mutex_unlock(&g_pool.mu);
      return NULL;
    }
    seen = g_pool.gen;
    orc_task_fn fn = g_pool.fn;
    void *arg = g_pool.arg;
    const int nw = g_pool.n;
    pthread_mutex_unlock(&g_pool.mu);
    fn(arg, w, nw);
    pthread_mutex_lock(&g_pool.mu);
    g_pool.completed++;
    pthread_cond_broadcast(&g_pool.cv_done);
    pthread_mutex_unlock(&g_pool.mu);
  }
}

static void pool_stop(void) {
  if (!g_pool_up) return;
  pthread_mutex_lock(&g_pool.mu);
  g_pool.quit = 1;
  pthread_cond_broadcast(&g_pool.cv_work);
  pthread_mutex_unlock(&g_pool.mu);
  for (int i = 1; i < g_pool.n; ++i) pthread_join(g_pool.thr[i], NULL);
  free(g_pool.thr);
  pthread_mutex_destroy(&g_pool.mu);
  pthread_cond_destroy(&g_pool.cv_work);
  pthread_cond_destroy(&g_pool.cv_done);
  g_pool_up = 0;
}

static void pool_start(int n) {
  if (n < 1) n = 1;
  g_pool.n = n;
  g_pool.thr = (pthread_t *)calloc((size_t)n, sizeof(pthread_t));
  pthread_mutex_init(&g_pool.mu, NULL);
  pthread_cond_init(&g_pool.cv_work, NULL);
  pthread_cond_init(&g_pool.cv_done, NULL);
  g_pool.gen = 0;
  g_pool.completed = 0;
  g_pool.quit = 0;
  for (int i = 1; i < n; ++i) {
    worker_arg *a = (worker_arg *)malloc(sizeof(worker_arg));
    a->w = i;
    pthread_create(&g_pool.thr[i], NULL, worker_main, a);
  }
  g_pool_up = 1;
}

void orc_set_threads(int n) {
  pthread_mutex_lock(&g_pool_init_mu);
  pool_stop();
  pool_start(n);
  pthread_mutex_unlock(&g_pool_init_mu);
}

int orc_threads(void) {
  if (!g_pool_up) {
    long c = sysconf(_SC_NPROCESSORS_ONLN);
    orc_set_threads(c > 0 ? (int)c : 1);
  }
  return g_pool.n;
}

void orc_run(orc_task_fn fn, void *arg) {
  const int n = orc_threads();
  if (n == 1) {
    fn(arg, 0, 1);
    return;
  }
  pthread_mutex_lock(&g_pool.mu);
  g_pool.fn = fn;
  g_pool.arg = arg;
  const long target = g_pool.completed + (n - 1);
  g_pool.gen++;
  pthread_cond_broadcast(&g_pool.cv_work);
  pthread_mutex_unlock(&g_pool.mu);
  fn(arg, 0, n);
  pthread_mutex_lock(&g_pool.mu);
  while (g_pool.completed < target) pthread_cond_wait(&g_pool.cv_done, &g_pool.mu);
  pthread_mutex_unlock(&g_pool.mu);
}

void orc_range(int64_t n, int w, int nw, int64_t *lo, int64_t *hi) {
  const int64_t chunk = (n + nw - 1) / nw;
  int64_t a = chunk * w;
  if (a > n) a = n;
  int64_t b = a + chunk;
  if (b > n) b = n;
  *lo = a;
  *hi = b;
}
