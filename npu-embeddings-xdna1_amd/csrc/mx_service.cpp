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
//
// A lane keeps two chunks in flight on its stream: chunk j's ids and mask
// are copied into one of two pinned host slots and sent by DMA, embedded
// without the closing wait (mx_encoder_embed_async), and its pooled rows and
// the stream's refusal flag come back into the same slot; while chunk j + 1
// runs, the host copies chunk j's rows out of the slot. Stream order keeps
// the lane's single set of device buffers safe; each slot's event says when
// its copies are done.
#include <atomic>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "mx_internal.hpp"

using mx::fail;

namespace {

// One of a lane's two pinned host slots: a chunk's ids and mask on their way
// in, its pooled rows and the refusal flag on their way back.
struct Slot {
  int32_t *ids = nullptr;
  float *mask = nullptr, *out = nullptr;
  int *flag = nullptr;
  hipEvent_t done = nullptr;
};

struct Lane {
  mx_encoder *enc = nullptr;
  bool own_enc = false;
  mx_stream *s = nullptr;
  int32_t *ids = nullptr;
  float *mask = nullptr, *out = nullptr;
  Slot slot[2];
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
    if (l.s) (void)hipStreamSynchronize(l.s->stream);
    for (Slot &sl : l.slot) {
      if (sl.ids) (void)hipHostFree(sl.ids);
      if (sl.mask) (void)hipHostFree(sl.mask);
      if (sl.out) (void)hipHostFree(sl.out);
      if (sl.flag) (void)hipHostFree(sl.flag);
      if (sl.done) (void)hipEventDestroy(sl.done);
    }
    if (l.ids) (void)hipFree(l.ids);
    if (l.mask) (void)hipFree(l.mask);
    if (l.out) (void)hipFree(l.out);
    if (l.s) mx_stream_destroy(l.s);
    if (l.own_enc) mx_encoder_destroy(l.enc);
  }
  delete svc;
}

int host_alloc(void **p, size_t bytes) {
  const hipError_t e = hipHostMalloc(p, bytes ? bytes : 1, hipHostMallocDefault);
  return e == hipSuccess ? MX_OK : mx::hip_fail(e, "embed_service: pinned host buffer");
}

// A lane's two pinned slots.
int make_slots(mx_embed_service *svc, Lane &l) {
  const size_t in = static_cast<size_t>(svc->batch * svc->seq) * 4;
  const size_t outb = static_cast<size_t>(svc->batch * svc->hidden) * 4;
  int rc = MX_OK;
  for (Slot &sl : l.slot) {
    if (!rc) rc = host_alloc((void **)&sl.ids, in);
    if (!rc) rc = host_alloc((void **)&sl.mask, in);
    if (!rc) rc = host_alloc((void **)&sl.out, outb);
    if (!rc) rc = host_alloc((void **)&sl.flag, 2 * sizeof(int));
    if (!rc) {
      const hipError_t e = hipEventCreateWithFlags(&sl.done, hipEventDisableTiming);
      if (e != hipSuccess) rc = mx::hip_fail(e, "embed_service: event");
    }
  }
  return rc;
}

// Queue rows [base, base + take) of the request through lane l into slot sl:
// the inputs into the pinned slot and on to the device, the embed, the
// pooled rows and the refusal flag back into the slot, then the slot's event.
int issue(mx_embed_service *svc, Lane &l, Slot &sl, const int32_t *ids, const float *mask,
          int64_t base, int64_t take) {
  const int64_t S = svc->seq, d = svc->hidden;
  const size_t in = static_cast<size_t>(take * S) * 4;
  std::memcpy(sl.ids, ids + base * S, in);
  std::memcpy(sl.mask, mask + base * S, in);
  int rc = mx_copy_h2d(l.s, l.ids, sl.ids, in);
  if (!rc) rc = mx_copy_h2d(l.s, l.mask, sl.mask, in);
  if (!rc) rc = mx_encoder_embed_async(l.enc, l.s, l.ids, l.mask, take, S, l.out);
  if (!rc) rc = mx_copy_d2h(l.s, sl.out, l.out, static_cast<size_t>(take * d) * 4);
  if (!rc) rc = mx_copy_d2h(l.s, sl.flag, l.s->err_dev, 2 * sizeof(int));
  if (!rc) {
    const hipError_t e = hipEventRecord(sl.done, l.s->stream);
    if (e != hipSuccess) rc = mx::hip_fail(e, "embed_service: event record");
  }
  return rc;
}

// Wait for slot sl's chunk and copy its rows out; a refusal the chunk's
// kernels raised is read (and cleared) by mx_sync, which names it. The packed
// row total that came back with the flag is the stream's next tile hint, as
// mx_sync would have set it.
int collect(mx_embed_service *svc, Lane &l, Slot &sl, int64_t base, int64_t take, float *out) {
  const hipError_t e = hipEventSynchronize(sl.done);
  if (e != hipSuccess) return mx::hip_fail(e, "embed_service: waiting for a chunk");
  if (sl.flag[0]) return mx_sync(l.s);
  if (sl.flag[1] > 0) l.s->last_rows = sl.flag[1];
  const int64_t d = svc->hidden;
  std::memcpy(out + base * d, sl.out, static_cast<size_t>(take * d) * 4);
  return MX_OK;
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
    if (!rc) rc = make_slots(svc, l);
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
  std::atomic<size_t> next{0};
  std::atomic<bool> stop{false};
  std::mutex mu;
  int first_rc = MX_OK;
  std::string first_msg;
  auto record = [&](int rc) {
    std::lock_guard<std::mutex> lk(mu);
    if (first_rc == MX_OK) {
      first_rc = rc;
      first_msg = mx_last_error();
    }
    stop.store(true, std::memory_order_relaxed);
  };
  // A lane's loop: queue chunk j into one slot, then collect the chunk in the
  // other slot (queued the round before) while chunk j runs.
  auto worker = [&](Lane &l) {
    long prev = -1;  // the job in slot cur ^ 1, not yet collected
    int cur = 0;
    for (size_t j = next++; j < jobs.size(); j = next++) {
      if (stop.load(std::memory_order_relaxed)) break;
      int rc = issue(svc, l, l.slot[cur], ids_host, mask_host, jobs[j].first, jobs[j].second);
      if (!rc && prev >= 0)
        rc = collect(svc, l, l.slot[cur ^ 1], jobs[prev].first, jobs[prev].second, out_host);
      if (rc) {
        record(rc);
        prev = -1;
        break;
      }
      prev = static_cast<long>(j);
      cur ^= 1;
    }
    if (prev >= 0 && !stop.load(std::memory_order_relaxed)) {
      const int rc =
          collect(svc, l, l.slot[cur ^ 1], jobs[prev].first, jobs[prev].second, out_host);
      if (rc) record(rc);
    }
    // Drain the lane; a refusal of a chunk never collected is read and
    // cleared here too (the call has already failed).
    const int rc = mx_sync(l.s);
    if (rc) record(rc);
  };
  if (svc->lanes.size() == 1 || jobs.size() <= 1) {
    worker(svc->lanes[0]);
  } else {
    std::vector<std::thread> threads;
    for (size_t i = 1; i < svc->lanes.size(); ++i)
      threads.emplace_back([&, i] { worker(svc->lanes[i]); });
    worker(svc->lanes[0]);
    for (auto &t : threads) t.join();
  }
  if (first_rc) return fail(first_rc, first_msg);
  return MX_OK;
}

}  // extern "C"
