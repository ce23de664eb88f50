// mx_encoder.cpp -- the encoder stack on the GPU: BertEncoder::run's layer loop
// (bert_encoder.cpp:1419-1598) and the pre-LN ViT/Whisper body (vit/encoder.cpp:
// 222-431, whisper/encoder.cpp:114-213) with every activation resident in HBM,
// plus EmbedService::chunk's embed -> run -> pool (embed_service.cpp:29-64).
//
// HBM layout of one run over M = B*S rows (d = hidden, f = ffn):
//   x     fp32 [M, d]   residual stream (the caller's buffer, updated in place)
//   xb    bf16 [M, d]   LayerNorm output, the next GEMM's A operand
//   qkv   bf16 [M, 3d]  fused Q|K|V (Q pre-scaled by the packer)
//   ctx   bf16 [M, d]   attention output
//   proj  bf16 [M, d]   attn-out / FFN-down result, narrowed once (BERT; the
//                       residual-fused LayerNorm reads it; the array path's
//                       bf16-C convention, kernels/narrow_f32_bf16.cc)
//   up    bf16 [M, f]   FFN-up with bias and GELU fused into the GEMM
// Weights are [N, K] bf16 panels; biases and LayerNorm parameters fp32.
#include "mx_internal.hpp"
#include "mx_kernels.hpp"

#include <cctype>
#include <cstring>
#include <set>
#include <string>
#include <vector>

namespace mx {
std::set<std::string> placed_ops();
}

using namespace mx;

namespace {

struct LayerW {
  uint16_t *w[4] = {nullptr, nullptr, nullptr, nullptr};  // qkv, attn_out, ffn_up, ffn_down
  float *b[4] = {nullptr, nullptr, nullptr, nullptr};
  float *ln[4] = {nullptr, nullptr, nullptr, nullptr};  // ln1.w, ln1.b, ln2.w, ln2.b
};

enum Cat { CAT_GEMM = 0, CAT_ATTN = 1, CAT_LN = 2, CAT_OTHER = 3 };
// GEMM sites of a layer, in the order of mx_timings.gemm_site_*.
enum Site { SITE_QKV = 0, SITE_AO = 1, SITE_UP = 2, SITE_DOWN = 3 };

}  // namespace

struct mx_encoder {
  mx_ctx *ctx = nullptr;
  mx_encoder_desc desc{};
  std::vector<LayerW> layers;
  float *emb_ln[2] = {nullptr, nullptr};
  float *fin_ln[2] = {nullptr, nullptr};
  float *word = nullptr, *pos = nullptr, *type = nullptr;
  // workspace
  int64_t ws_rows = 0, ws_batch = 0;
  uint16_t *xb = nullptr, *qkv = nullptr, *ctxb = nullptr, *up = nullptr;
  uint16_t *proj = nullptr;
  float *emb = nullptr, *add_mask = nullptr;
  int32_t *kv_len = nullptr;
  // timing
  bool timing = false;
  std::vector<hipEvent_t> events;
  std::vector<int> ev_cat;
  size_t ev_used = 0;
  hipEvent_t ev_all[2] = {nullptr, nullptr};
  double gemm_flop = 0, attn_flop = 0;
  double site_flop[4] = {0, 0, 0, 0};
};

namespace {

void free_dev(void *&p) {
  if (p) (void)hipFree(p);
  p = nullptr;
}

template <typename T>
void free_dev(T *&p) {
  if (p) (void)hipFree(p);
  p = nullptr;
}

int dev_alloc(void **p, size_t bytes, const char *what) {
  const hipError_t e = hipMalloc(p, bytes);
  return e == hipSuccess ? MX_OK : hip_fail(e, what);
}

int ensure_ws(mx_encoder *enc, int64_t B, int64_t S) {
  const int64_t rows = B * S;
  const int64_t d = enc->desc.hidden, f = enc->desc.ffn;
  if (rows > enc->ws_rows) {
    free_dev(enc->xb);
    free_dev(enc->qkv);
    free_dev(enc->ctxb);
    free_dev(enc->up);
    free_dev(enc->proj);
    free_dev(enc->emb);
    enc->ws_rows = 0;
    int rc = dev_alloc((void **)&enc->xb, rows * d * 2, "workspace xb");
    if (!rc) rc = dev_alloc((void **)&enc->qkv, rows * 3 * d * 2, "workspace qkv");
    if (!rc) rc = dev_alloc((void **)&enc->ctxb, rows * d * 2, "workspace ctx");
    if (!rc) rc = dev_alloc((void **)&enc->up, rows * f * 2, "workspace up");
    if (!rc) rc = dev_alloc((void **)&enc->proj, rows * d * 2, "workspace proj");
    if (!rc) rc = dev_alloc((void **)&enc->emb, rows * d * 4, "workspace emb");
    if (rc) return rc;
    enc->ws_rows = rows;
  }
  if (B > enc->ws_batch || rows > enc->ws_rows) {
    free_dev(enc->add_mask);
    free_dev(enc->kv_len);
    enc->ws_batch = 0;
    int rc = dev_alloc((void **)&enc->add_mask, rows * 4, "workspace mask");
    if (!rc) rc = dev_alloc((void **)&enc->kv_len, B * 4, "workspace kv_len");
    if (rc) return rc;
    enc->ws_batch = B;
  }
  return MX_OK;
}

// Timing brackets: one event pair per launch when timing is on.
struct Bracket {
  mx_encoder *enc;
  hipStream_t s;
  int cat;
  Bracket(mx_encoder *e, hipStream_t st, int c) : enc(e), s(st), cat(c) {
    if (!enc->timing) return;
    if (enc->ev_used + 2 > enc->events.size()) {
      for (int i = 0; i < 64; ++i) {
        hipEvent_t ev;
        if (hipEventCreate(&ev) != hipSuccess) return;
        enc->events.push_back(ev);
        enc->ev_cat.push_back(0);
      }
    }
    (void)hipEventRecord(enc->events[enc->ev_used], s);
  }
  ~Bracket() {
    if (!enc->timing || enc->ev_used + 2 > enc->events.size()) return;
    (void)hipEventRecord(enc->events[enc->ev_used + 1], s);
    enc->ev_cat[enc->ev_used] = cat;
    enc->ev_used += 2;
  }
};

int check_placement() {
  const std::set<std::string> ops = placed_ops();
  if (ops.empty()) return MX_OK;
  static const char *need[] = {"gemm", "attn", "softm", "layn", "gelu"};
  std::string missing;
  for (const char *c : need)
    if (!ops.count(c)) missing += missing.empty() ? c : std::string(", ") + c;
  if (missing.empty()) return MX_OK;
  return fail(MX_E_INVALID,
              "encoder run: --npu-ops places only part of the encoder layer on the GPU (" +
                  missing +
                  " stay on the host). The fused GPU stack runs every op of the layer; "
                  "a partial placement is served op by op through mx_gemm / mx_attention "
                  "/ mx_softmax_rows / mx_layernorm / mx_gelu.");
}

int gemm_l(mx_encoder *enc, mx_stream *s, int site, const uint16_t *A, int64_t M, int64_t K,
           const uint16_t *Wt, int64_t N, const float *bias, int epi, const float *resid,
           void *C, int c_dtype) {
  Bracket br(enc, s->stream, CAT_GEMM + 16 * site);
  enc->gemm_flop += 2.0 * M * N * K;
  enc->site_flop[site] += 2.0 * M * N * K;
  return gemm_checked(s, A, M, K, K, Wt, N, bias, epi, resid, C, c_dtype, N);
}

int ln_l(mx_encoder *enc, mx_stream *s, const void *x, int x_dt, const void *y, int y_dt,
         const float *g, const float *b, int64_t rows, float *of, uint16_t *ob) {
  Bracket br(enc, s->stream, CAT_LN);
  const hipError_t e = mxk::layernorm(x, x_dt == MX_BF16, y, y_dt == MX_BF16, g, b,
                                      enc->desc.ln_eps, rows, enc->desc.hidden, of, ob, s->stream);
  return e == hipSuccess ? MX_OK : hip_fail(e, "layernorm launch");
}

int attn_l(mx_encoder *enc, mx_stream *s, int64_t B, int64_t S, const float *mask,
           const int32_t *kv_len) {
  Bracket br(enc, s->stream, CAT_ATTN);
  const int64_t d = enc->desc.hidden;
  enc->attn_flop += 4.0 * B * enc->desc.heads * (double)S * S * enc->desc.head_dim;
  return attention_checked(s, enc->qkv, 3 * d, B, S, enc->desc.heads, enc->desc.head_dim,
                           enc->desc.attn_scale, mask, kv_len, enc->ctxb, d);
}

int run_bert(mx_encoder *enc, mx_stream *s, float *x, const float *mask, const int32_t *kvl,
             int64_t B, int64_t S) {
  const int64_t M = B * S, d = enc->desc.hidden, f = enc->desc.ffn;
  const int epi = enc->desc.gelu == MX_GELU_ERF ? MX_EPI_GELU_ERF : MX_EPI_GELU_POLY;
  int rc = ln_l(enc, s, x, MX_F32, nullptr, MX_F32, enc->emb_ln[0], enc->emb_ln[1], M, x, enc->xb);
  for (size_t l = 0; !rc && l < enc->layers.size(); ++l) {
    const LayerW &w = enc->layers[l];
    rc = gemm_l(enc, s, SITE_QKV, enc->xb, M, d, w.w[0], 3 * d, w.b[0], MX_EPI_NONE, nullptr, enc->qkv,
                MX_BF16);
    if (!rc) rc = attn_l(enc, s, B, S, mask, kvl);
    if (!rc)
      rc = gemm_l(enc, s, SITE_AO, enc->ctxb, M, d, w.w[1], d, w.b[1], MX_EPI_NONE, nullptr, enc->proj,
                  MX_BF16);
    if (!rc) rc = ln_l(enc, s, x, MX_F32, enc->proj, MX_BF16, w.ln[0], w.ln[1], M, x, enc->xb);
    if (!rc)
      rc = gemm_l(enc, s, SITE_UP, enc->xb, M, d, w.w[2], f, w.b[2], epi, nullptr, enc->up, MX_BF16);
    if (!rc)
      rc = gemm_l(enc, s, SITE_DOWN, enc->up, M, f, w.w[3], d, w.b[3], MX_EPI_NONE, nullptr, enc->proj,
                  MX_BF16);
    if (!rc) rc = ln_l(enc, s, x, MX_F32, enc->proj, MX_BF16, w.ln[2], w.ln[3], M, x, enc->xb);
  }
  return rc;
}

int run_preln(mx_encoder *enc, mx_stream *s, float *x, const float *mask, const int32_t *kvl,
              int64_t B, int64_t S) {
  const int64_t M = B * S, d = enc->desc.hidden, f = enc->desc.ffn;
  const int epi = enc->desc.gelu == MX_GELU_POLY ? MX_EPI_GELU_POLY : MX_EPI_GELU_ERF;
  int rc = MX_OK;
  for (size_t l = 0; !rc && l < enc->layers.size(); ++l) {
    const LayerW &w = enc->layers[l];
    rc = ln_l(enc, s, x, MX_F32, nullptr, MX_F32, w.ln[0], w.ln[1], M, nullptr, enc->xb);
    if (!rc)
      rc = gemm_l(enc, s, SITE_QKV, enc->xb, M, d, w.w[0], 3 * d, w.b[0], MX_EPI_NONE, nullptr, enc->qkv,
                  MX_BF16);
    if (!rc) rc = attn_l(enc, s, B, S, mask, kvl);
    if (!rc)
      rc = gemm_l(enc, s, SITE_AO, enc->ctxb, M, d, w.w[1], d, w.b[1], MX_EPI_NONE, x, x, MX_F32);
    if (!rc) rc = ln_l(enc, s, x, MX_F32, nullptr, MX_F32, w.ln[2], w.ln[3], M, nullptr, enc->xb);
    if (!rc)
      rc = gemm_l(enc, s, SITE_UP, enc->xb, M, d, w.w[2], f, w.b[2], epi, nullptr, enc->up, MX_BF16);
    if (!rc) rc = gemm_l(enc, s, SITE_DOWN, enc->up, M, f, w.w[3], d, w.b[3], MX_EPI_NONE, x, x, MX_F32);
  }
  if (!rc) rc = ln_l(enc, s, x, MX_F32, nullptr, MX_F32, enc->fin_ln[0], enc->fin_ln[1], M, x, nullptr);
  return rc;
}

int run_impl(mx_encoder *enc, mx_stream *s, float *x, const float *mask, const int32_t *kvl,
             int64_t B, int64_t S) {
  return enc->desc.arch == MX_ARCH_BERT ? run_bert(enc, s, x, mask, kvl, B, S)
                                        : run_preln(enc, s, x, mask, kvl, B, S);
}

int begin_timing(mx_encoder *enc, mx_stream *s) {
  enc->ev_used = 0;
  enc->gemm_flop = enc->attn_flop = 0;
  for (double &f : enc->site_flop) f = 0;
  if (!enc->timing) return MX_OK;
  for (auto &ev : enc->ev_all)
    if (!ev && hipEventCreate(&ev) != hipSuccess) return fail(MX_E_DEVICE, "hipEventCreate");
  (void)hipEventRecord(enc->ev_all[0], s->stream);
  return MX_OK;
}

void end_timing(mx_encoder *enc, mx_stream *s) {
  if (enc->timing) (void)hipEventRecord(enc->ev_all[1], s->stream);
}

const char *kGemmNames[4] = {"qkv", "attn_out", "ffn_up", "ffn_down"};

}  // namespace

extern "C" {

int mx_encoder_create(mx_ctx *ctx, const mx_encoder_desc *desc, mx_encoder **out) {
  clear_error();
  if (!ctx || !desc || !out) return fail(MX_E_INVALID, "encoder_create: null argument");
  *out = nullptr;
  const mx_encoder_desc &d = *desc;
  if (d.arch != MX_ARCH_BERT && d.arch != MX_ARCH_PRELN)
    return fail(MX_E_INVALID, "encoder_create: unknown arch " + std::to_string(d.arch));
  if (d.layers <= 0 || d.hidden <= 0 || d.heads <= 0 || d.head_dim <= 0 || d.ffn <= 0)
    return fail(MX_E_INVALID, "encoder_create: zero dimension");
  if (d.heads * d.head_dim != d.hidden)
    return fail(MX_E_INVALID, "encoder_create: " + std::to_string(d.heads) + " heads x " +
                                  std::to_string(d.head_dim) + " is not hidden " +
                                  std::to_string(d.hidden));
  if (d.hidden % 8 || d.ffn % 8)
    return fail(MX_E_INVALID, "encoder_create: hidden and ffn must be multiples of 8");
  if (d.head_dim != 32 && d.head_dim != 64)
    return fail(MX_E_UNSUPPORTED, "encoder_create: head_dim " + std::to_string(d.head_dim) +
                                      " (the attention kernel is built for 32 and 64)");
  if (d.gelu != MX_GELU_POLY && d.gelu != MX_GELU_ERF)
    return fail(MX_E_INVALID, "encoder_create: gelu must be MX_GELU_POLY or MX_GELU_ERF");
  if (!(d.ln_eps >= 0.0f)) return fail(MX_E_INVALID, "encoder_create: bad ln_eps");
  int rc = use_device(ctx);
  if (rc) return rc;
  auto *e = new mx_encoder();
  e->ctx = ctx;
  e->desc = d;
  e->layers.resize(static_cast<size_t>(d.layers));
  *out = e;
  return MX_OK;
}

void mx_encoder_destroy(mx_encoder *enc) {
  if (!enc) return;
  if (use_device(enc->ctx) == MX_OK) {
    for (auto &l : enc->layers) {
      for (auto &p : l.w) free_dev(p);
      for (auto &p : l.b) free_dev(p);
      for (auto &p : l.ln) free_dev(p);
    }
    for (auto &p : enc->emb_ln) free_dev(p);
    for (auto &p : enc->fin_ln) free_dev(p);
    free_dev(enc->word);
    free_dev(enc->pos);
    free_dev(enc->type);
    free_dev(enc->xb);
    free_dev(enc->qkv);
    free_dev(enc->ctxb);
    free_dev(enc->up);
    free_dev(enc->proj);
    free_dev(enc->emb);
    free_dev(enc->add_mask);
    free_dev(enc->kv_len);
    for (auto ev : enc->events) (void)hipEventDestroy(ev);
    for (auto ev : enc->ev_all)
      if (ev) (void)hipEventDestroy(ev);
  }
  delete enc;
}

int mx_encoder_set(mx_encoder *enc, const char *name_c, const void *host, int dtype,
                   int64_t count) {
  clear_error();
  if (!enc || !name_c || !host) return fail(MX_E_INVALID, "encoder_set: null argument");
  int rc = use_device(enc->ctx);
  if (rc) return rc;
  const std::string name(name_c);
  const int64_t d = enc->desc.hidden, f = enc->desc.ffn;
  auto put_f32 = [&](float *&dst, int64_t want) -> int {
    if (dtype != MX_F32) return fail(MX_E_INVALID, name + ": must be MX_F32");
    if (count != want)
      return fail(MX_E_INVALID, name + ": " + std::to_string(count) + " values, " +
                                    std::to_string(want) + " wanted");
    free_dev(dst);
    int r = dev_alloc((void **)&dst, want * 4, name.c_str());
    if (r) return r;
    const hipError_t e = hipMemcpy(dst, host, want * 4, hipMemcpyHostToDevice);
    return e == hipSuccess ? MX_OK : hip_fail(e, name.c_str());
  };
  if (name.rfind("layer.", 0) == 0) {
    size_t p = 6;
    int64_t L = 0;
    bool digits = false;
    while (p < name.size() && std::isdigit(static_cast<unsigned char>(name[p]))) {
      L = L * 10 + (name[p] - '0');
      ++p;
      digits = true;
    }
    if (!digits || p >= name.size() || name[p] != '.')
      return fail(MX_E_INVALID, "encoder_set: cannot read the layer index of '" + name + "'");
    if (L >= enc->desc.layers)
      return fail(MX_E_INVALID, "encoder_set: '" + name + "' names layer " + std::to_string(L) +
                                    " of a " + std::to_string(enc->desc.layers) + "-layer stack");
    const std::string rest = name.substr(p + 1);
    LayerW &w = enc->layers[static_cast<size_t>(L)];
    const int64_t K[4] = {d, d, d, f}, N[4] = {3 * d, d, f, d};
    for (int i = 0; i < 4; ++i) {
      if (rest == kGemmNames[i]) {
        if (count != K[i] * N[i])
          return fail(MX_E_INVALID, name + ": " + std::to_string(count) + " values, a [" +
                                        std::to_string(K[i]) + ", " + std::to_string(N[i]) +
                                        "] operand wanted");
        uint16_t *panel = nullptr;
        int r = stage_panel(enc->ctx, host, dtype, K[i], N[i], &panel);
        if (r) return r;
        free_dev(w.w[i]);
        w.w[i] = panel;
        return MX_OK;
      }
      if (rest == std::string(kGemmNames[i]) + ".bias") return put_f32(w.b[i], N[i]);
    }
    if (rest == "ln1.weight") return put_f32(w.ln[0], d);
    if (rest == "ln1.bias") return put_f32(w.ln[1], d);
    if (rest == "ln2.weight") return put_f32(w.ln[2], d);
    if (rest == "ln2.bias") return put_f32(w.ln[3], d);
    return fail(MX_E_INVALID, "encoder_set: unknown tensor '" + name + "'");
  }
  if (name == "embeddings.ln.weight") return put_f32(enc->emb_ln[0], d);
  if (name == "embeddings.ln.bias") return put_f32(enc->emb_ln[1], d);
  if (name == "final_ln.weight") return put_f32(enc->fin_ln[0], d);
  if (name == "final_ln.bias") return put_f32(enc->fin_ln[1], d);
  if (name == "embeddings.word") {
    if (enc->desc.vocab <= 0) return fail(MX_E_INVALID, "embeddings.word: desc.vocab is 0");
    return put_f32(enc->word, enc->desc.vocab * d);
  }
  if (name == "embeddings.position") {
    if (enc->desc.max_pos <= 0) return fail(MX_E_INVALID, "embeddings.position: desc.max_pos is 0");
    return put_f32(enc->pos, enc->desc.max_pos * d);
  }
  if (name == "embeddings.token_type") {
    if (count < d || count % d)
      return fail(MX_E_INVALID, "embeddings.token_type: a whole number of rows of hidden");
    free_dev(enc->type);
    int r = dev_alloc((void **)&enc->type, count * 4, name.c_str());
    if (r) return r;
    const hipError_t e = hipMemcpy(enc->type, host, count * 4, hipMemcpyHostToDevice);
    return e == hipSuccess ? MX_OK : hip_fail(e, name.c_str());
  }
  return fail(MX_E_INVALID, "encoder_set: unknown tensor '" + name + "'");
}

int mx_encoder_ready(mx_encoder *enc) {
  if (!enc) return fail(MX_E_INVALID, "encoder_ready: null encoder");
  for (size_t l = 0; l < enc->layers.size(); ++l) {
    const LayerW &w = enc->layers[l];
    const std::string p = "layer." + std::to_string(l) + ".";
    for (int i = 0; i < 4; ++i) {
      if (!w.w[i]) return fail(MX_E_STATE, "encoder: " + p + kGemmNames[i] + " was never set");
      if (!w.b[i])
        return fail(MX_E_STATE, "encoder: " + p + kGemmNames[i] + ".bias was never set");
    }
    static const char *lnn[4] = {"ln1.weight", "ln1.bias", "ln2.weight", "ln2.bias"};
    for (int i = 0; i < 4; ++i)
      if (!w.ln[i]) return fail(MX_E_STATE, "encoder: " + p + lnn[i] + " was never set");
  }
  if (enc->desc.arch == MX_ARCH_BERT) {
    if (!enc->emb_ln[0] || !enc->emb_ln[1])
      return fail(MX_E_STATE, "encoder: embeddings.ln.weight/bias were never set");
  } else if (!enc->fin_ln[0] || !enc->fin_ln[1]) {
    return fail(MX_E_STATE, "encoder: final_ln.weight/bias were never set");
  }
  return MX_OK;
}

int mx_encoder_run(mx_encoder *enc, mx_stream *s, float *x_io, const float *add_mask,
                   const int32_t *kv_len, int64_t B, int64_t S) {
  clear_error();
  if (!enc || !s || !x_io) return fail(MX_E_INVALID, "encoder_run: null argument");
  if (B <= 0 || S <= 0) return fail(MX_E_INVALID, "encoder_run: empty batch");
  int rc = check_placement();
  if (!rc) rc = mx_encoder_ready(enc);
  if (!rc) rc = use_device(enc->ctx);
  if (!rc) rc = ensure_ws(enc, B, S);
  if (!rc) rc = begin_timing(enc, s);
  if (rc) return rc;
  rc = run_impl(enc, s, x_io, add_mask, kv_len, B, S);
  end_timing(enc, s);
  return rc;
}

int mx_encoder_embed(mx_encoder *enc, mx_stream *s, const int32_t *ids, const float *attn_mask,
                     int64_t B, int64_t S, float *out) {
  clear_error();
  if (!enc || !s || !ids || !attn_mask || !out)
    return fail(MX_E_INVALID, "encoder_embed: null argument");
  if (enc->desc.arch != MX_ARCH_BERT)
    return fail(MX_E_INVALID, "encoder_embed: the text path is the BERT encoder's");
  if (!enc->word || !enc->pos || !enc->type)
    return fail(MX_E_STATE, "encoder_embed: embeddings.word/position/token_type not set");
  if (S > enc->desc.max_pos)
    return fail(MX_E_INVALID, "encoder_embed: seq " + std::to_string(S) + " exceeds the " +
                                  std::to_string(enc->desc.max_pos) + " position embeddings");
  int rc = use_device(enc->ctx);
  if (!rc) rc = check_placement();
  if (!rc) rc = mx_encoder_ready(enc);
  if (!rc) rc = ensure_ws(enc, B, S);
  if (!rc) rc = begin_timing(enc, s);
  if (rc) return rc;
  {
    Bracket br(enc, s->stream, CAT_OTHER);
    hipError_t e = mxk::embed_sum(ids, B, S, enc->desc.hidden, enc->word, enc->desc.vocab,
                                  enc->pos, enc->type, enc->emb, s->err_dev, s->stream);
    if (e == hipSuccess)
      e = mxk::mask_build(attn_mask, B, S, enc->add_mask, enc->kv_len, s->stream);
    if (e != hipSuccess) return hip_fail(e, "embed launch");
  }
  rc = run_impl(enc, s, enc->emb, enc->add_mask, enc->kv_len, B, S);
  if (rc) return rc;
  {
    Bracket br(enc, s->stream, CAT_OTHER);
    const hipError_t e =
        mxk::pool_rows(enc->emb, attn_mask, B, S, enc->desc.hidden, enc->desc.cls_pool,
                       enc->desc.l2_normalize, out, s->err_dev, s->stream);
    if (e != hipSuccess) return hip_fail(e, "pool launch");
  }
  end_timing(enc, s);
  int flags = 0;
  rc = take_data_error(s, &flags);
  if (rc) return rc;
  if (flags & 1)
    return fail(MX_E_DATA, "encoder_embed: a token id is outside [0, " +
                               std::to_string(enc->desc.vocab) + ")");
  if (flags & 2) return fail(MX_E_DATA, "CLS pooling on a sequence whose first token is masked");
  return MX_OK;
}

int mx_encoder_set_timing(mx_encoder *enc, int on) {
  if (!enc) return fail(MX_E_INVALID, "encoder_set_timing: null encoder");
  enc->timing = on != 0;
  return MX_OK;
}

int mx_encoder_timings(mx_encoder *enc, mx_timings *out) {
  clear_error();
  if (!enc || !out) return fail(MX_E_INVALID, "encoder_timings: null argument");
  std::memset(out, 0, sizeof *out);
  out->gemm_flop = enc->gemm_flop;
  out->attn_flop = enc->attn_flop;
  for (int i = 0; i < 4; ++i) out->gemm_site_flop[i] = enc->site_flop[i];
  if (!enc->timing) return MX_OK;
  int rc = use_device(enc->ctx);
  if (rc) return rc;
  for (size_t i = 0; i + 1 < enc->ev_used; i += 2) {
    hipError_t e = hipEventSynchronize(enc->events[i + 1]);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, enc->events[i], enc->events[i + 1]);
    if (e != hipSuccess) return hip_fail(e, "hipEventElapsedTime");
    if (enc->ev_cat[i] % 16 == CAT_GEMM) {
      const int site = enc->ev_cat[i] / 16;
      out->gemm_site_ms[site] += ms;
      ++out->gemm_site_launches[site];
    }
    switch (enc->ev_cat[i] % 16) {
      case CAT_GEMM: out->gemm_ms += ms; ++out->gemm_launches; break;
      case CAT_ATTN: out->attn_ms += ms; ++out->attn_launches; break;
      case CAT_LN: out->ln_ms += ms; ++out->ln_launches; break;
      default: out->other_ms += ms; ++out->other_launches; break;
    }
  }
  if (enc->ev_all[0] && enc->ev_all[1]) {
    float ms = 0.0f;
    if (hipEventSynchronize(enc->ev_all[1]) == hipSuccess &&
        hipEventElapsedTime(&ms, enc->ev_all[0], enc->ev_all[1]) == hipSuccess)
      out->total_ms = ms;
  }
  return MX_OK;
}

}  // extern "C"
