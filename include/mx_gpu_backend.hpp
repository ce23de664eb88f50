/* mx_gpu_backend.hpp -- the C++ face of mx_encoder.h for the reference
 * runtime (C++17). Every failure becomes std::runtime_error("gpu: <reason>"),
 * the reference's convention for a refusal (runtime/src/entry.cpp:74-77
 * prints it and exits 2); every handle is released by its destructor.
 *
 *   Backend    npu::Device (runtime/include/runtime/device.hpp:28-39): the
 *              context on one GPU
 *   Lane       one --pipeline lane (run_setup.hpp:778-874): a stream; sync()
 *              is the synchronous completion Design::dispatch_only gives
 *   Buffer     a device allocation (Design's A/C slots, design.hpp:199-263)
 *   Container  npue::File (runtime/src/model.cpp:214-380): a mapped .npue
 *   Encoder    BertEncoder (bert_encoder.cpp:1419-1598) built from a
 *              container, with EmbedService::chunk's embed
 *              (embed_service.cpp:29-64) from token ids on
 *   EmbedService  EmbedService::embed (embed_service.cpp:66-108) minus the
 *              tokenizer: host ids and masks in, host rows out, over lanes
 */
#ifndef MX_GPU_BACKEND_HPP
#define MX_GPU_BACKEND_HPP

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>

#include "mx_encoder.h"

namespace mxgpu {

inline void check(int rc) {
  if (rc != MX_OK) throw std::runtime_error(std::string("gpu: ") + mx_last_error());
}

class Backend {
 public:
  explicit Backend(int device = 0) { check(mx_create(device, &ctx_)); }
  ~Backend() { mx_destroy(ctx_); }
  Backend(const Backend &) = delete;
  Backend &operator=(const Backend &) = delete;
  mx_ctx *get() const { return ctx_; }

 private:
  mx_ctx *ctx_ = nullptr;
};

class Lane {
 public:
  explicit Lane(Backend &b) { check(mx_stream_create(b.get(), &s_)); }
  ~Lane() { mx_stream_destroy(s_); }
  Lane(const Lane &) = delete;
  Lane &operator=(const Lane &) = delete;
  mx_stream *get() const { return s_; }
  void sync() { check(mx_sync(s_)); }
  void to_device(void *dev, const void *host, size_t bytes) {
    check(mx_copy_h2d(s_, dev, host, bytes));
  }
  void to_host(void *host, const void *dev, size_t bytes) {
    check(mx_copy_d2h(s_, host, dev, bytes));
  }

 private:
  mx_stream *s_ = nullptr;
};

class Buffer {
 public:
  Buffer(Backend &b, size_t bytes) : ctx_(b.get()) { check(mx_alloc(ctx_, bytes, &p_)); }
  ~Buffer() {
    if (p_) (void)mx_free(ctx_, p_);
  }
  Buffer(const Buffer &) = delete;
  Buffer &operator=(const Buffer &) = delete;
  void *get() const { return p_; }

 private:
  mx_ctx *ctx_ = nullptr;
  void *p_ = nullptr;
};

class Container {
 public:
  explicit Container(const std::string &path) { check(mx_npue_open(path.c_str(), &f_)); }
  ~Container() { mx_npue_close(f_); }
  Container(const Container &) = delete;
  Container &operator=(const Container &) = delete;
  const mx_npue *get() const { return f_; }
  // File::config_string (model.cpp:374-379): the value's text; throws when
  // absent. mx_npue_config returns the value's full length, so a value longer
  // than the first buffer is read again into one of that size.
  std::string config(const std::string &key) const {
    std::string v(256, '\0');
    int n = mx_npue_config(f_, key.c_str(), &v[0], v.size());
    if (n < 0) check(n);
    if (static_cast<size_t>(n) >= v.size()) {
      v.assign(static_cast<size_t>(n) + 1, '\0');
      n = mx_npue_config(f_, key.c_str(), &v[0], v.size());
      if (n < 0) check(n);
    }
    v.resize(static_cast<size_t>(n));
    return v;
  }

 private:
  mx_npue *f_ = nullptr;
};

class Encoder {
 public:
  // setup_encoder + set_model_shape + stage_all for a BERT container
  // (run_setup.hpp:483-877, app_state.hpp:440-550): ready on return.
  Encoder(Backend &b, const Container &c) { check(mx_encoder_from_npue(b.get(), c.get(), &e_)); }
  ~Encoder() { mx_encoder_destroy(e_); }
  Encoder(const Encoder &) = delete;
  Encoder &operator=(const Encoder &) = delete;
  mx_encoder *get() const { return e_; }
  // EmbedService::chunk minus the tokenizer: ids int32 [B, S] and the 1/0
  // mask fp32 [B, S] (device) -> pooled, L2-normalised fp32 [B, hidden]
  // (device). Returns when the rows are ready, as chunk() returns them.
  void embed(Lane &lane, const int32_t *ids, const float *mask, int64_t B, int64_t S,
             float *out) {
    check(mx_encoder_embed(e_, lane.get(), ids, mask, B, S, out));
  }
  // The same embed queued without its closing wait (no counterpart in the
  // reference): the rows are ready, and a data refusal is thrown, at the
  // lane's next sync().
  void embed_async(Lane &lane, const int32_t *ids, const float *mask, int64_t B, int64_t S,
                   float *out) {
    check(mx_encoder_embed_async(e_, lane.get(), ids, mask, B, S, out));
  }

 private:
  mx_encoder *e_ = nullptr;
};

class EmbedService {
 public:
  // make_service's lanes (embed_service.cpp:110-119): `lanes` workers, each
  // an encoder clone on a stream of its own, chunks of `batch` sequences of
  // length `seq`. `enc` must outlive the service.
  EmbedService(Encoder &enc, int lanes, int64_t batch, int64_t seq) {
    check(mx_embed_service_create(enc.get(), lanes, batch, seq, &svc_));
  }
  ~EmbedService() { mx_embed_service_destroy(svc_); }
  EmbedService(const EmbedService &) = delete;
  EmbedService &operator=(const EmbedService &) = delete;
  mx_embed_service *get() const { return svc_; }
  // n sequences: ids int32 [n, seq] and the 1/0 masks fp32 [n, seq] (host)
  // -> pooled, L2-normalised fp32 [n, hidden] (host). The first failing
  // chunk's refusal is thrown; the others are not run.
  void embed(const int32_t *ids, const float *mask, int64_t n, float *out) {
    check(mx_embed_service_embed(svc_, ids, mask, n, out));
  }

 private:
  mx_embed_service *svc_ = nullptr;
};

}  // namespace mxgpu

#endif  // MX_GPU_BACKEND_HPP
