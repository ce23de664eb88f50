// mx_service.cpp -- EmbedService::embed (runtime/src/server/embed_service.cpp:
// 12-108) over the GPU backend, minus the tokenizer: a request of n sequences
// (token ids and 1/0 masks, host memory) is cut into chunks of `batch`
// sequences (plan(), :12-27, with no compiled tiers: every chunk is `batch`
// but the last), and the chunks are taken by `lanes` workers, each with its
// own stream, device buffers and encoder workspace over the one set of
// weights (the reference's --pipeline lanes, run_setup.hpp:778-874). Each
// chunk is embed sum -> encoder -> pool (chunk(), :29-64) into its rows of
// the output. The first failing chunk stops the others and its error is the
// call's (:80-92).
#include <atomic>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "mx_internal.hpp"

using mx::fail;

namespace {

struct Lane {
  mx_encoder *enc = nullptr;
  bool own_enc = false;
  mx_stream *s = nullptr;
  int32_t *ids = nullptr;
  float *mask = nullptr, *out = nullptr;
};

}  // namespace

struct mx_embed_service {
  mx_encoder *lead = nullptr;
  mx_ctx *ctx = nullptr;
  int64_t batch = 0, seq = 0, hidden = 0;
  std::vector<Lane> lanes;
};

namespace {

void release(mx_embed_service *svc) {
  for (Lane &l : svc->lanes) {
    if (l.ids) (void)hipFree(l.ids);
    if (l.mask) (void)hipFree(l.mask);
    if (l.out) (void)hipFree(l.out);
    if (l.s) mx_stream_destroy(l.s);
    if (l.own_enc) mx_encoder_destroy(l.enc);
  }
  delete svc;
}

// One chunk: rows [base, base + take) of the request through lane l.
int chunk(mx_embed_service *svc, Lane &l, const int32_t *ids, const float *mask, int64_t base,
          int64_t take, float *out) {
  const int64_t S = svc->seq, d = svc->hidden;
  int rc = mx_copy_h2d(l.s, l.ids, ids + base * S, static_cast<size_t>(take * S) * 4);
  if (!rc) rc = mx_copy_h2d(l.s, l.mask, mask + base * S, static_cast<size_t>(take * S) * 4);
  if (!rc) rc = mx_encoder_embed(l.enc, l.s, l.ids, l.mask, take, S, l.out);
  if (!rc) rc = mx_copy_d2h(l.s, out + base * d, l.out, static_cast<size_t>(take * d) * 4);
  if (!rc) rc = mx_sync(l.s);
  return rc;
}

}  // namespace

extern "C" {

int mx_embed_service_create(mx_encoder *enc, int lanes, int64_t batch, int64_t seq,
                            mx_embed_service **out) {
  mx::clear_error();
  if (!enc || !out) return fail(MX_E_INVALID, "embed_service: null argument");
  *out = nullptr;
  if (lanes < 1 || lanes > 64) return fail(MX_E_INVALID, "embed_service: lanes must be 1..64");
  if (batch < 1 || seq < 1) return fail(MX_E_INVALID, "embed_service: batch and seq must be >= 1");
  mx_encoder *probe = nullptr;
  int rc = mx_encoder_clone(enc, &probe);  // checks the encoder is complete
  if (rc) return rc;
  auto *svc = new mx_embed_service;
  svc->lead = enc;
  svc->ctx = mx::encoder_ctx(enc);
  svc->batch = batch;
  svc->seq = seq;
  svc->hidden = mx::encoder_hidden(enc);
  svc->lanes.resize(static_cast<size_t>(lanes));
  for (int i = 0; i < lanes && !rc; ++i) {
    Lane &l = svc->lanes[static_cast<size_t>(i)];
    if (i == 0) {
      l.enc = probe;
      l.own_enc = true;
    } else {
      rc = mx_encoder_clone(enc, &l.enc);
      l.own_enc = rc == MX_OK;
    }
    if (!rc) rc = mx_stream_create(svc->ctx, &l.s);
    if (!rc) rc = mx_alloc(svc->ctx, static_cast<size_t>(batch * seq) * 4, (void **)&l.ids);
    if (!rc) rc = mx_alloc(svc->ctx, static_cast<size_t>(batch * seq) * 4, (void **)&l.mask);
    if (!rc) rc = mx_alloc(svc->ctx, static_cast<size_t>(batch * svc->hidden) * 4, (void **)&l.out);
  }
  if (rc) {
    const std::string msg = mx_last_error();
    release(svc);
    return fail(rc, msg);
  }
  *out = svc;
  return MX_OK;
}

void mx_embed_service_destroy(mx_embed_service *svc) {
  if (svc) release(svc);
}

int mx_embed_service_embed(mx_embed_service *svc, const int32_t *ids_host, const float *mask_host,
                           int64_t n, float *out_host) {
  mx::clear_error();
  if (!svc || !ids_host || !mask_host || !out_host)
    return fail(MX_E_INVALID, "embed_service_embed: null argument");
  if (n < 0) return fail(MX_E_INVALID, "embed_service_embed: negative count");
  std::vector<std::pair<int64_t, int64_t>> jobs;
  for (int64_t base = 0; base < n; base += svc->batch)
    jobs.emplace_back(base, n - base < svc->batch ? n - base : svc->batch);
  if (svc->lanes.size() == 1 || jobs.size() <= 1) {
    for (const auto &j : jobs) {
      const int rc = chunk(svc, svc->lanes[0], ids_host, mask_host, j.first, j.second, out_host);
      if (rc) return rc;
    }
    return MX_OK;
  }
  std::atomic<size_t> next{0};
  std::atomic<bool> stop{false};
  std::mutex mu;
  int first_rc = MX_OK;
  std::string first_msg;
  auto worker = [&](Lane &l) {
    for (size_t j = next++; j < jobs.size(); j = next++) {
      if (stop.load(std::memory_order_relaxed)) return;
      const int rc = chunk(svc, l, ids_host, mask_host, jobs[j].first, jobs[j].second, out_host);
      if (rc) {
        std::lock_guard<std::mutex> lk(mu);
        if (first_rc == MX_OK) {
          first_rc = rc;
          first_msg = mx_last_error();
        }
        stop.store(true, std::memory_order_relaxed);
        return;
      }
    }
  };
  std::vector<std::thread> threads;
  for (size_t i = 1; i < svc->lanes.size(); ++i)
    threads.emplace_back([&, i] { worker(svc->lanes[i]); });
  worker(svc->lanes[0]);
  for (auto &t : threads) t.join();
  if (first_rc) return fail(first_rc, first_msg);
  return MX_OK;
}

}  // extern "C"
