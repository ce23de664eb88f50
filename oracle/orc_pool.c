/*
 * orc_pool.c -- the oracle's persistent worker pools. TEST INFRASTRUCTURE.
 *
 * Restates app::Pool (runtime/include/runtime/pool.hpp:18-39,
 * runtime/src/pool.cpp:28-110): N persistent workers, a generation counter and
 * a CUMULATIVE completion count (a count-down released waiters early in the
 * reference's history, pool.cpp:62-81). run(f) calls f(w, nw) once on every
 * worker, worker 0 being the caller, and returns when all have finished.
 *
 * One process-wide pool (orc_set_threads), plus, for the reference's
 * --pipeline lanes (runtime/include/runtime/run_setup.hpp:465-477: one Pool of
 * threads / pipeline workers per lane), a pool of the calling thread's own
 * (orc_lane_begin / orc_lane_end): while a thread holds one, its orc_run calls
 * use it, so concurrent lanes never share workers.
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
static __thread orc_pool_t *tl_pool = NULL;

typedef struct {
  orc_pool_t *pool;
  int w;
} worker_arg;

static void *worker_main(void *p) {
  orc_pool_t *pool = ((worker_arg *)p)->pool;
  const int w = ((worker_arg *)p)->w;
  free(p);
  long seen = 0;
  for (;;) {
    pthread_mutex_lock(&pool->mu);
    while (!pool->quit && pool->gen == seen) pthread_cond_wait(&pool->cv_work, &pool->mu);
    if (pool->quit) {
      pthread_mutex_unlock(&pool->mu);
      return NULL;
    }
    seen = pool->gen;
    orc_task_fn fn = pool->fn;
    void *arg = pool->arg;
    const int nw = pool->n;
    pthread_mutex_unlock(&pool->mu);
    fn(arg, w, nw);
    pthread_mutex_lock(&pool->mu);
    pool->completed++;
    pthread_cond_broadcast(&pool->cv_done);
    pthread_mutex_unlock(&pool->mu);
  }
}

static void pool_stop(orc_pool_t *pool) {
  pthread_mutex_lock(&pool->mu);
  pool->quit = 1;
  pthread_cond_broadcast(&pool->cv_work);
  pthread_mutex_unlock(&pool->mu);
  for (int i = 1; i < pool->n; ++i) pthread_join(pool->thr[i], NULL);
  free(pool->thr);
  pthread_mutex_destroy(&pool->mu);
  pthread_cond_destroy(&pool->cv_work);
  pthread_cond_destroy(&pool->cv_done);
}

static void pool_start(orc_pool_t *pool, int n) {
  if (n < 1) n = 1;
  pool->n = n;
  pool->thr = (pthread_t *)calloc((size_t)n, sizeof(pthread_t));
  pthread_mutex_init(&pool->mu, NULL);
  pthread_cond_init(&pool->cv_work, NULL);
  pthread_cond_init(&pool->cv_done, NULL);
  pool->gen = 0;
  pool->completed = 0;
  pool->quit = 0;
  for (int i = 1; i < n; ++i) {
    worker_arg *a = (worker_arg *)malloc(sizeof(worker_arg));
    a->pool = pool;
    a->w = i;
    pthread_create(&pool->thr[i], NULL, worker_main, a);
  }
}

void orc_set_threads(int n) {
  pthread_mutex_lock(&g_pool_init_mu);
  if (g_pool_up) pool_stop(&g_pool);
  pool_start(&g_pool, n);
  g_pool_up = 1;
  pthread_mutex_unlock(&g_pool_init_mu);
}

int orc_threads(void) {
  if (tl_pool) return tl_pool->n;
  if (!g_pool_up) {
    long c = sysconf(_SC_NPROCESSORS_ONLN);
    orc_set_threads(c > 0 ? (int)c : 1);
  }
  return g_pool.n;
}

int orc_lane_begin(int n) {
  if (tl_pool) return -1;
  orc_pool_t *p = (orc_pool_t *)calloc(1, sizeof(orc_pool_t));
  if (!p) return -1;
  pool_start(p, n);
  tl_pool = p;
  return 0;
}

void orc_lane_end(void) {
  if (!tl_pool) return;
  pool_stop(tl_pool);
  free(tl_pool);
  tl_pool = NULL;
}

void orc_run(orc_task_fn fn, void *arg) {
  const int n = orc_threads();
  if (n == 1) {
    fn(arg, 0, 1);
    return;
  }
  orc_pool_t *pool = tl_pool ? tl_pool : &g_pool;
  pthread_mutex_lock(&pool->mu);
  pool->fn = fn;
  pool->arg = arg;
  const long target = pool->completed + (n - 1);
  pool->gen++;
  pthread_cond_broadcast(&pool->cv_work);
  pthread_mutex_unlock(&pool->mu);
  fn(arg, 0, n);
  pthread_mutex_lock(&pool->mu);
  while (pool->completed < target) pthread_cond_wait(&pool->cv_done, &pool->mu);
  pthread_mutex_unlock(&pool->mu);
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
