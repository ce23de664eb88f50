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
//
// An int8 container (every GEMM operand int8 with its wscale and asmooth)
// runs the W8A8 datapath of the reference's int8 design: each GEMM's A is
// quantised per row into
//   xq    int8 [M, max(d, f)]  the quantised A operand
//   sa    fp32 [M]             its row scales
// by the residual LayerNorm itself (add_norm_quant) or by a quantise pass
// over ctx / up, and the GEMM dequantises in its epilogue; the other buffers
// keep their roles (xb is then unused).
#include "mx_internal.hpp"
#include "mx_kernels.hpp"

#include <cctype>
#include <cstring>
#include <mutex>
#include <set>
#include <string>
#include <vector>

using namespace mx;

namespace mx {
mx_ctx *encoder_ctx(const mx_encoder *enc);
int64_t encoder_hidden(const mx_encoder *enc);
}  // namespace mx

namespace {

struct LayerW {
  uint16_t *w[4] = {nullptr, nullptr, nullptr, nullptr};  // qkv, attn_out, ffn_up, ffn_down
  float *b[4] = {nullptr, nullptr, nullptr, nullptr};
  float *ln[4] = {nullptr, nullptr, nullptr, nullptr};  // ln1.w, ln1.b, ln2.w, ln2.b
  // int8 operands: [N, K] int8 panel, wscale [N], ias = 1/asmooth [K]
  int8_t *wq[4] = {nullptr, nullptr, nullptr, nullptr};
  float *ws[4] = {nullptr, nullptr, nullptr, nullptr};
  float *ias[4] = {nullptr, nullptr, nullptr, nullptr};
  // The gated FFN fused into FFN-up's epilogue: FFN-up's operand (bf16 or
  // int8), bias and wscale with their 2f rows in glu_interleave's order,
  // built from the tensors of weight generation glu_gen.
  uint16_t *wg = nullptr;
  int8_t *wqg = nullptr;
  float *bg = nullptr, *wsg = nullptr;
  uint64_t glu_gen = 0;
};

enum Cat { CAT_GEMM = 0, CAT_ATTN = 1, CAT_LN = 2, CAT_OTHER = 3 };
// GEMM sites of a layer, in the order of mx_timings.gemm_site_*.
enum Site { SITE_QKV = 0, SITE_AO = 1, SITE_UP = 2, SITE_DOWN = 3 };

// The device buffers one embed / run works in (the HBM layout above).
struct Work {
  uint16_t *xb = nullptr, *qkv = nullptr, *ctxb = nullptr, *up = nullptr;
  uint16_t *proj = nullptr;
  float *emb = nullptr, *add_mask = nullptr;
  int8_t *xq = nullptr;  // int8 datapath: quantised A and its row scales
  float *sa = nullptr;
  uint16_t *glu = nullptr;  // gated FFN: lo * act(hi), [M, f] bf16
  int32_t *kv_len = nullptr;
  // token packing: seq_start [B + 1] then attention's launch order [B], and
  // each packed row's position [M]
  int32_t *seq_start = nullptr, *row_pos = nullptr;
};

}  // namespace

struct mx_encoder {
  mx_ctx *ctx = nullptr;
  mx_encoder_desc desc{};
  bool owns_weights = true;  // false for a lane clone, which borrows its parent's
  // Lane clones borrow the owner's weight pointers. While any clone is alive
  // the owner's weights neither change (set / set_panel refuse) nor go away:
  // destroying the owner first frees only its workspace and leaves the rest
  // to the last clone's destroy. Guarded by g_clone_mu.
  mx_encoder *owner = nullptr;  // a clone's owner
  int live_clones = 0;          // an owner's clones not yet destroyed
  bool orphaned = false;        // an owner destroyed while clones were alive
  // Bumped by every tensor set: the fused gated FFN's interleaved copies are
  // current while their glu_gen equals it.
  uint64_t wgen = 1;
  bool fuse_glu = true;  // the gated FFN in FFN-up's epilogue where it can run
  std::vector<LayerW> layers;
  float *emb_ln[2] = {nullptr, nullptr};
  float *fin_ln[2] = {nullptr, nullptr};
  float *word = nullptr, *pos = nullptr, *type = nullptr;
  // workspace: the encoder's own (sized by ensure_ws), or for one
  // mx_encoder_embed_static call the carved static scratch
  int64_t ws_rows = 0, ws_batch = 0, ws_mask_rows = 0;
  Work work;
  // RoPE: the frequencies when the container gives them ("rope.inv_freq"),
  // and the device cos/sin tables [rope_rows, head_dim], built on first use.
  std::vector<float> rope_inv;
  float *rope_cos = nullptr, *rope_sin = nullptr;
  int64_t rope_rows = 0;
  bool i8 = false;       // set by mx_encoder_ready: every GEMM operand is int8
  // The array designs' narrowed C (mx_encoder_set_narrowed_c): every GEMM's
  // accumulator rounded to bf16 before its bias / dequantisation.
  bool narrow_c = false;
  bool ws_wide = false;  // the workspace holds proj / up / glu in fp32
  // Token packing (embed): seq_start [B + 1] and each packed row's position
  // (work.seq_start, work.row_pos).
  bool packing = true;
  // CLS pooling: the last layer's attention-out, FFN and LayerNorms over the
  // sequences' first rows only (mx_encoder_set_cls_pruning)
  bool prune_cls = true;
  // The last packed plan read back (seq_start[0..B]) and its sum of squared
  // lengths: the attention work of a packed pass.
  std::vector<int32_t> plan_host;
  double packed_sq = 0.0;
  // A packed pass whose row total stays on the device (no host wait in the
  // middle of the call): the launches over live_bound rows (the B * S the
  // workspace holds) take live -- the total's device address, and as the GEMM
  // tile hint the stream's last total read with its refusal flag.
  mx::Live live;
  int64_t live_bound = 0;
  // timing
  bool timing = false;
  std::vector<hipEvent_t> events;
  std::vector<int> ev_cat;
  size_t ev_used = 0;
  hipEvent_t ev_all[2] = {nullptr, nullptr};
  double gemm_flop = 0, attn_flop = 0;
  double site_flop[4] = {0, 0, 0, 0};
  // front ends (ViT / Whisper) and the ViT head
  uint16_t *patch_w = nullptr, *head_w = nullptr, *conv_w[2] = {nullptr, nullptr};
  float *patch_b = nullptr, *head_b = nullptr, *conv_b[2] = {nullptr, nullptr};
  float *cls_tok = nullptr, *front_pos = nullptr;
  int64_t fw_batch = 0;  // front workspace sized for this batch
  uint16_t *f_rows = nullptr, *f_cls = nullptr, *f_mel = nullptr, *f_out1 = nullptr;
  float *f_patch = nullptr, *f_x = nullptr;
};

namespace {

std::mutex g_clone_mu;

template <typename T>
void free_dev(T *&p) {
  if (p) (void)hipFree(p);
  p = nullptr;
}

int dev_alloc(void **p, size_t bytes, const char *what) {
  const hipError_t e = dev_malloc(p, bytes);
  return e == hipSuccess ? MX_OK : hip_fail(e, what);
}

int ensure_ws_rows(mx_encoder *enc, int64_t rows, int64_t B);
int ensure_mask_ws(mx_encoder *enc, int64_t B, int64_t rows);

// proj, up and the gated product in fp32: the int8 datapath (dequantise_c's
// C, dequant_act_quant's activation) and a narrowed C (from_bf16(c) + bias).
bool wide_acts(const mx_encoder *enc) { return enc->i8 || enc->narrow_c; }

int ensure_ws(mx_encoder *enc, int64_t B, int64_t S) {
  const int64_t rows = B * S;
  if (rows > enc->ws_rows || (enc->i8 && !enc->work.xq) || (wide_acts(enc) && !enc->ws_wide)) {
    const int64_t want = rows > enc->ws_rows ? rows : enc->ws_rows;
    return ensure_ws_rows(enc, want, B);
  }
  return ensure_mask_ws(enc, B, rows);
}

// Work already queued (mx_encoder_embed_async) may still use the workspace a
// regrowth frees: wait for the device first.
int drain_workspace(const mx_encoder *enc) {
  if (!enc->work.xb && !enc->work.add_mask) return MX_OK;
  const hipError_t e = hipDeviceSynchronize();
  return e == hipSuccess ? MX_OK : hip_fail(e, "workspace regrowth: draining queued work");
}

int ensure_ws_rows(mx_encoder *enc, int64_t rows, int64_t B) {
  const int64_t d = enc->desc.hidden, f = enc->desc.ffn;
  {
    const int drc = drain_workspace(enc);
    if (drc) return drc;
    free_dev(enc->work.xb);
    free_dev(enc->work.qkv);
    free_dev(enc->work.ctxb);
    free_dev(enc->work.up);
    free_dev(enc->work.proj);
    free_dev(enc->work.emb);
    free_dev(enc->work.xq);
    free_dev(enc->work.sa);
    free_dev(enc->work.glu);
    enc->ws_rows = 0;
    const int64_t fu = enc->desc.gated_ffn ? 2 * f : f;
    int rc = dev_alloc((void **)&enc->work.xb, rows * d * 2, "workspace xb");
    if (!rc) rc = dev_alloc((void **)&enc->work.qkv, rows * 3 * d * 2, "workspace qkv");
    if (!rc) rc = dev_alloc((void **)&enc->work.ctxb, rows * d * 2, "workspace ctx");
    // int8: FFN-up's activation stays fp32 up to its quantiser; a narrowed C
    // keeps from_bf16(c) + bias in fp32
    const int64_t ab = wide_acts(enc) ? 4 : 2;
    if (!rc) rc = dev_alloc((void **)&enc->work.up, rows * fu * ab, "workspace up");
    if (!rc && enc->desc.gated_ffn)
      rc = dev_alloc((void **)&enc->work.glu, rows * f * ab, "workspace gated");
    // int8: the attention-out / FFN-down results stay fp32 (dequantise_c's C)
    if (!rc) rc = dev_alloc((void **)&enc->work.proj, rows * d * ab, "workspace proj");
    if (!rc) rc = dev_alloc((void **)&enc->work.emb, rows * d * 4, "workspace emb");
    if (!rc && enc->i8)
      rc = dev_alloc((void **)&enc->work.xq, rows * (d > f ? d : f), "workspace xq");
    if (!rc && enc->i8) rc = dev_alloc((void **)&enc->work.sa, rows * 4, "workspace sa");
    if (rc) return rc;
    enc->ws_rows = rows;
    enc->ws_wide = ab == 4;
  }
  return ensure_mask_ws(enc, B, rows);
}

// The mask ([B, S] fp32) and kv_len ([B]) buffers, sized by their own
// capacities: a longer sequence at the same batch needs a larger mask.
int ensure_mask_ws(mx_encoder *enc, int64_t B, int64_t rows) {
  if (B > enc->ws_batch || rows > enc->ws_mask_rows) {
    const int64_t nb = B > enc->ws_batch ? B : enc->ws_batch;
    const int64_t nr = rows > enc->ws_mask_rows ? rows : enc->ws_mask_rows;
    const int drc = drain_workspace(enc);
    if (drc) return drc;
    free_dev(enc->work.add_mask);
    free_dev(enc->work.kv_len);
    free_dev(enc->work.seq_start);
    free_dev(enc->work.row_pos);
    enc->ws_batch = enc->ws_mask_rows = 0;
    int rc = dev_alloc((void **)&enc->work.add_mask, nr * 4, "workspace mask");
    if (!rc) rc = dev_alloc((void **)&enc->work.kv_len, nb * 4, "workspace kv_len");
    // seq_start [B + 1], then attention's launch order [B].
    if (!rc) rc = dev_alloc((void **)&enc->work.seq_start, (2 * nb + 1) * 4, "workspace seq_start");
    if (!rc) rc = dev_alloc((void **)&enc->work.row_pos, nr * 4, "workspace row_pos");
    if (rc) return rc;
    enc->ws_batch = nb;
    enc->ws_mask_rows = nr;
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

// The live rows of a launch over M rows: the pass's device-side count when M
// is the pass's row bound, else M itself.
mx::Live live_of(const mx_encoder *enc, int64_t M) {
  return M == enc->live_bound ? enc->live : mx::Live{};
}

int gemm_l(mx_encoder *enc, mx_stream *s, int site, const uint16_t *A, int64_t M, int64_t K,
           const uint16_t *Wt, int64_t N, const float *bias, int epi, const float *resid,
           void *C, int c_dtype) {
  Bracket br(enc, s->stream, CAT_GEMM + 16 * site);
  enc->gemm_flop += 2.0 * M * N * K;
  enc->site_flop[site] += 2.0 * M * N * K;
  return gemm_checked(s, A, M, K, K, Wt, N, bias, epi, resid, C, c_dtype, N, live_of(enc, M));
}

int ln_l(mx_encoder *enc, mx_stream *s, const void *x, int x_dt, const void *y, int y_dt,
         const float *g, const float *b, int64_t rows, float *of, uint16_t *ob) {
  Bracket br(enc, s->stream, CAT_LN);
  const hipError_t e =
      mxk::layernorm(x, x_dt == MX_BF16, y, y_dt == MX_BF16, g, b, enc->desc.ln_eps, rows,
                     enc->desc.hidden, of, ob, s->stream, live_of(enc, rows).dev);
  return e == hipSuccess ? MX_OK : hip_fail(e, "layernorm launch");
}

// The int8 datapath's three steps: the GEMM on the quantised A, the residual
// LayerNorm that quantises its output for the next GEMM, and the quantise pass
// over an activation another kernel produced (ctx, up).
int gemm_i8_l(mx_encoder *enc, mx_stream *s, int site, int64_t M, int64_t K, const int8_t *Wq,
              const float *ws, int64_t N, const float *bias, int epi, const float *resid,
              void *C, int c_dtype) {
  Bracket br(enc, s->stream, CAT_GEMM + 16 * site);
  enc->gemm_flop += 2.0 * M * N * K;
  enc->site_flop[site] += 2.0 * M * N * K;
  return gemm_i8_checked(s, enc->work.xq, enc->work.sa, M, K, K, Wq, ws, N, bias, epi, resid, C,
                         c_dtype, N, live_of(enc, M));
}

int lnq_l(mx_encoder *enc, mx_stream *s, const float *x, const void *y, int y_dt, const float *g,
          const float *b, int64_t rows, float *of, const float *ias) {
  Bracket br(enc, s->stream, CAT_LN);
  return layernorm_i8_checked(s, x, y, y_dt, g, b, enc->desc.ln_eps, rows, enc->desc.hidden, of,
                              ias, enc->work.xq, enc->work.sa, live_of(enc, rows));
}

int quant_l(mx_encoder *enc, mx_stream *s, const void *a, int a_dtype, int64_t rows, int64_t K,
            const float *ias) {
  Bracket br(enc, s->stream, CAT_OTHER);
  return quantise_checked(s, a, a_dtype, K, rows, K, ias, enc->work.xq, K, enc->work.sa,
                          live_of(enc, rows));
}

// RoPE tables for positions [0, S), built on the host once (double angles,
// as apply_rope_qkv builds them) and kept on the device.
int ensure_rope(mx_encoder *enc, int64_t S) {
  if (S <= enc->rope_rows) return MX_OK;
  const int64_t hd = enc->desc.head_dim;
  std::vector<float> c(static_cast<size_t>(S * hd)), sn(static_cast<size_t>(S * hd));
  rope_tables_host(S, hd, enc->desc.rope_theta, enc->rope_inv.empty() ? nullptr : enc->rope_inv.data(),
                   c.data(), sn.data());
  free_dev(enc->rope_cos);
  free_dev(enc->rope_sin);
  enc->rope_rows = 0;
  int rc = dev_alloc((void **)&enc->rope_cos, c.size() * 4, "rope table");
  if (!rc) rc = dev_alloc((void **)&enc->rope_sin, sn.size() * 4, "rope table");
  if (rc) return rc;
  hipError_t e = upload(enc->rope_cos, c.data(), c.size() * 4);
  if (e == hipSuccess) e = upload(enc->rope_sin, sn.data(), sn.size() * 4);
  if (e != hipSuccess) return hip_fail(e, "rope table upload");
  enc->rope_rows = S;
  return MX_OK;
}

int rope_l(mx_encoder *enc, mx_stream *s, int64_t B, int64_t S, int64_t M,
           const int32_t *row_pos) {
  Bracket br(enc, s->stream, CAT_OTHER);
  return rope_checked(s, enc->work.qkv, 3 * enc->desc.hidden, B, S, enc->desc.heads,
                      enc->desc.head_dim, enc->rope_cos, enc->rope_sin, M, row_pos,
                      live_of(enc, M));
}

int glu_l(mx_encoder *enc, mx_stream *s, int64_t M, int in_dtype, int out_dtype) {
  Bracket br(enc, s->stream, CAT_OTHER);
  return glu_checked(s, enc->work.up, in_dtype, enc->work.glu, out_dtype, M, enc->desc.ffn,
                     enc->desc.gated_ffn, live_of(enc, M));
}

// Whether FFN-up can carry the gated FFN in its epilogue: whole 64-row
// groups of the interleaved operand (f % 32 == 0) on the LDS-pipelined bf16
// kernel (K a multiple of 32, at least 128). The int8 datapath keeps FFN-up's
// activation in fp32 up to its quantiser (dequant_act_quant), which the
// fused epilogue's bf16 C does not, so it runs the GEMM and the GLU apart.
bool glu_fusable(const mx_encoder *enc) {
  const int64_t d = enc->desc.hidden, f = enc->desc.ffn;
  return enc->desc.gated_ffn != MX_GATED_NONE && f % 32 == 0 && !enc->i8 && d % 32 == 0 &&
         d >= 128;
}

// The interleaved FFN-up copies of every layer, when stale (owning encoder
// only; a clone runs the copies it was cloned with, or the unfused pair).
int ensure_glu_operands(mx_encoder *enc) {
  if (!enc->owns_weights || !enc->fuse_glu || !glu_fusable(enc)) return MX_OK;
  const int64_t d = enc->desc.hidden, f = enc->desc.ffn;
  bool synced = false;
  SetupStream st;
  for (LayerW &w : enc->layers) {
    if (w.glu_gen == enc->wgen) continue;
    if (!synced) {  // the source tensors may still be in flight
      const int rc = use_device(enc->ctx);
      if (rc) return rc;
      const hipError_t e = hipDeviceSynchronize();
      if (e != hipSuccess) return hip_fail(e, "gated FFN interleave");
      synced = true;
    }
    free_dev(w.wg);
    free_dev(w.wqg);
    free_dev(w.bg);
    free_dev(w.wsg);
    w.glu_gen = 0;
    int rc = dev_alloc((void **)&w.bg, 2 * f * 4, "gated FFN-up bias");
    hipError_t e = rc ? hipSuccess : mxk::glu_interleave(w.b[SITE_UP], w.bg, f, 4, st.s);
    if (!rc && e == hipSuccess) {
      if (enc->i8) {
        rc = dev_alloc((void **)&w.wqg, 2 * f * d, "gated FFN-up operand");
        if (!rc) rc = dev_alloc((void **)&w.wsg, 2 * f * 4, "gated FFN-up wscale");
        if (!rc) e = mxk::glu_interleave(w.wq[SITE_UP], w.wqg, f, d, st.s);
        if (!rc && e == hipSuccess) e = mxk::glu_interleave(w.ws[SITE_UP], w.wsg, f, 4, st.s);
      } else {
        rc = dev_alloc((void **)&w.wg, 2 * f * d * 2, "gated FFN-up operand");
        if (!rc) e = mxk::glu_interleave(w.w[SITE_UP], w.wg, f, d * 2, st.s);
      }
    }
    if (rc) return rc;
    if (e != hipSuccess) return hip_fail(e, "gated FFN interleave");
  }
  if (synced) {
    const hipError_t e = st.finish();
    if (e != hipSuccess) return hip_fail(e, "gated FFN interleave");
    for (LayerW &w : enc->layers) w.glu_gen = enc->wgen;
  }
  return MX_OK;
}

// FFN-up with the gated FFN fused: the layer's interleaved operand, C =
// enc->work.glu [M, f] bf16, the same values as the GEMM into enc->work.up and glu_l.
int gemm_glu_l(mx_encoder *enc, mx_stream *s, const LayerW &w, int64_t M) {
  Bracket br(enc, s->stream, CAT_GEMM + 16 * SITE_UP);
  const int64_t d = enc->desc.hidden, f = enc->desc.ffn;
  enc->gemm_flop += 2.0 * M * 2 * f * d;
  enc->site_flop[SITE_UP] += 2.0 * M * 2 * f * d;
  const int epi =
      enc->desc.gated_ffn == MX_GATED_SILU ? mxk::EPI_GLU_SILU : mxk::EPI_GLU_GELU;
  const mx::Live lv = live_of(enc, M);
  hipError_t e;
  if (enc->i8) {
    const mxk::GemmI8Args a{enc->work.xq, d,   w.wqg, M,       2 * f,         d,
                            enc->work.sa, w.wsg, w.bg, epi, nullptr, enc->work.glu,
                            1,            f,     lv.dev, lv.hint};
    e = mxk::gemm_i8(a, s->stream);
  } else {
    const mxk::GemmArgs a{enc->work.xb, d, w.wg, M, 2 * f, d, w.bg, epi, nullptr, enc->work.glu,
                          1,            f, lv.dev, lv.hint};
    e = mxk::gemm(a, s->stream);
  }
  return e == hipSuccess ? MX_OK : hip_fail(e, "gemm launch (FFN-up with the gated FFN)");
}

// The rows one pass runs over: M = B*S dense rows, or the packed rows of
// token packing (seq_start / row_pos non-null, M = seq_start[B]); order
// (nullable) is attention's launch order, longest sequence first.
struct Rows {
  int64_t M;
  const int32_t *seq_start = nullptr, *row_pos = nullptr, *order = nullptr;
};

// q_rows: 0 for every query, else only each sequence's first q_rows.
int attn_l(mx_encoder *enc, mx_stream *s, int64_t B, int64_t S, const float *mask,
           const int32_t *kv_len, const Rows *rows = nullptr, int64_t q_rows = 0) {
  Bracket br(enc, s->stream, CAT_ATTN);
  const int64_t d = enc->desc.hidden;
  // Packed rows: each sequence attends over its own kv_len rows only.
  const double sq = rows && rows->seq_start ? enc->packed_sq : (double)B * S * S;
  enc->attn_flop += 4.0 * enc->desc.heads * sq * enc->desc.head_dim;
  return attention_checked(s, enc->work.qkv, 3 * d, B, S, enc->desc.heads, enc->desc.head_dim,
                           enc->desc.attn_scale, mask, kv_len, enc->work.ctxb, d,
                           rows ? rows->seq_start : nullptr, rows ? rows->order : nullptr,
                           q_rows);
}

// One GEMM site of a layer on the encoder's datapath: bf16 A (A_bf) times
// the bf16 panel, or the quantised A in xq/sa times the int8 operand.
int site_gemm(mx_encoder *enc, mx_stream *s, const LayerW &w, int site, const uint16_t *A_bf,
              int64_t M, int64_t K, int64_t N, int epi, const float *resid, void *C,
              int c_dtype) {
  if (enc->narrow_c) epi |= MX_EPI_NARROW_C;
  if (enc->i8)
    return gemm_i8_l(enc, s, site, M, K, w.wq[site], w.ws[site], N, w.b[site], epi, resid, C,
                     c_dtype);
  return gemm_l(enc, s, site, A_bf, M, K, w.w[site], N, w.b[site], epi, resid, C, c_dtype);
}

// The LayerNorm ahead of a GEMM: x (+ y) normalised into out_f32, and the
// next GEMM's A -- bf16 into xb, or (int8) quantised with that GEMM's ias.
// ias_next null on the int8 datapath: nothing follows, no A is written.
int site_ln(mx_encoder *enc, mx_stream *s, float *x, const void *y, int y_dt, const float *g,
            const float *b, int64_t M, float *out_f32, const float *ias_next) {
  if (enc->i8 && ias_next) return lnq_l(enc, s, x, y, y_dt, g, b, M, out_f32, ias_next);
  return ln_l(enc, s, x, MX_F32, y, y_dt, g, b, M, out_f32, enc->i8 ? nullptr : enc->work.xb);
}

// The embedding LayerNorm ahead of the first layer (and the RoPE tables).
int bert_pre(mx_encoder *enc, mx_stream *s, float *x, int64_t S, const Rows &rows) {
  int rc = enc->desc.rope ? ensure_rope(enc, S) : MX_OK;
  if (!rc)
    rc = site_ln(enc, s, x, nullptr, MX_F32, enc->emb_ln[0], enc->emb_ln[1], rows.M, x,
                 enc->layers[0].ias[SITE_QKV]);
  return rc;
}

// Layer l of BertEncoder::run over the rows of one pass, in enc->work.
// The attention half of layer l over the pass's rows: QKV, RoPE, attention
// into enc->work.ctxb (q_rows: 0 for every query, else each sequence's first
// q_rows only).
int layer_attn(mx_encoder *enc, mx_stream *s, const float *mask, const int32_t *kvl, int64_t B,
               int64_t S, const Rows &rows, size_t l, int64_t q_rows = 0) {
  const int64_t M = rows.M, d = enc->desc.hidden;
  const LayerW &w = enc->layers[l];
  int rc = site_gemm(enc, s, w, SITE_QKV, enc->work.xb, M, d, 3 * d, MX_EPI_NONE, nullptr,
                     enc->work.qkv, MX_BF16);
  if (!rc && enc->desc.rope) rc = rope_l(enc, s, B, S, M, rows.row_pos);
  if (!rc) rc = attn_l(enc, s, B, S, mask, kvl, &rows, q_rows);
  return rc;
}

// The row-wise half of layer l over M rows -- x the residual stream and ctx
// the attention context (bf16), both [M, d]: attention-out, the residual
// LayerNorm, the FFN, the second LayerNorm. Each row's result depends on that
// row alone.
int layer_rows(mx_encoder *enc, mx_stream *s, float *x, const uint16_t *ctx, int64_t M,
               size_t l) {
  const int64_t d = enc->desc.hidden, f = enc->desc.ffn;
  const int epi = enc->desc.gelu == MX_GELU_ERF ? MX_EPI_GELU_ERF : MX_EPI_GELU_POLY;
  const size_t L = enc->layers.size();
  const bool gated = enc->desc.gated_ffn != MX_GATED_NONE;
  const int64_t fu = gated ? 2 * f : f;
  uint16_t *act = gated ? enc->work.glu : enc->work.up;  // FFN-down's A (bf16 datapath)
  const LayerW &w = enc->layers[l];
  const bool fused = gated && enc->fuse_glu && !enc->narrow_c && glu_fusable(enc) &&
                     w.glu_gen == enc->wgen && (enc->i8 ? w.wqg && w.wsg : w.wg != nullptr) &&
                     w.bg;
  int rc = enc->i8 ? quant_l(enc, s, ctx, MX_BF16, M, d, w.ias[SITE_AO]) : MX_OK;
  // proj: bf16 (the array path's C) or fp32 -- on the int8 datapath as
  // dequantise_c writes it (host_kernels.hpp:529-600), with a narrowed C as
  // from_bf16(c) + bias (bert_encoder.cpp:874-900)
  const int pdt = wide_acts(enc) ? MX_F32 : MX_BF16;
  if (!rc)
    rc = site_gemm(enc, s, w, SITE_AO, ctx, M, d, d, MX_EPI_NONE, nullptr, enc->work.proj, pdt);
  if (!rc) rc = site_ln(enc, s, x, enc->work.proj, pdt, w.ln[0], w.ln[1], M, x, w.ias[SITE_UP]);
  if (!rc && enc->i8) {
    // dequant_act_quant (host_kernels.hpp:405-522, bert_encoder.cpp:811-860):
    // FFN-up dequantised, biased and activated in fp32 (the gated halves
    // combined in fp32), then quantised per row from those fp32 values.
    rc = site_gemm(enc, s, w, SITE_UP, nullptr, M, d, fu, gated ? MX_EPI_NONE : epi, nullptr,
                   enc->work.up, MX_F32);
    if (!rc && gated) rc = glu_l(enc, s, M, MX_F32, MX_F32);
    if (!rc) rc = quant_l(enc, s, act, MX_F32, M, f, w.ias[SITE_DOWN]);
  } else if (!rc && fused) {
    rc = gemm_glu_l(enc, s, w, M);
  } else if (!rc && gated && enc->narrow_c) {
    // dequant_act_bf16's gated branch (bert_encoder.cpp:633-712): both halves
    // from_bf16(c) + bias in fp32, combined in fp32, rounded once to bf16.
    rc = site_gemm(enc, s, w, SITE_UP, enc->work.xb, M, d, fu, MX_EPI_NONE, nullptr,
                   enc->work.up, MX_F32);
    if (!rc) rc = glu_l(enc, s, M, MX_F32, MX_BF16);
  } else {
    if (!rc)
      rc = site_gemm(enc, s, w, SITE_UP, enc->work.xb, M, d, fu, gated ? MX_EPI_NONE : epi,
                     nullptr, enc->work.up, MX_BF16);
    if (!rc && gated) rc = glu_l(enc, s, M, MX_BF16, MX_BF16);
  }
  if (!rc)
    rc = site_gemm(enc, s, w, SITE_DOWN, act, M, f, d, MX_EPI_NONE, nullptr, enc->work.proj,
                   pdt);
  if (!rc)
    rc = site_ln(enc, s, x, enc->work.proj, pdt, w.ln[2], w.ln[3], M, x,
                 l + 1 < L ? enc->layers[l + 1].ias[SITE_QKV] : nullptr);
  return rc;
}

// Layer l of BertEncoder::run over the rows of one pass, in enc->work.
int bert_layer(mx_encoder *enc, mx_stream *s, float *x, const float *mask, const int32_t *kvl,
               int64_t B, int64_t S, const Rows &rows, size_t l) {
  int rc = layer_attn(enc, s, mask, kvl, B, S, rows, l);
  return rc ? rc : layer_rows(enc, s, x, enc->work.ctxb, rows.M, l);
}

// pooled (nullable): with CLS pooling and CLS pruning on, the last layer's
// attention computes each sequence's first query only (over all its keys)
// and its row-wise half runs over that first row only -- the other rows reach
// neither the pooled output nor a later layer -- gathered into the QKV
// buffer (free once attention has run) with the context rows in xb, and
// *pooled points at those B rows (row b for sequence b). Otherwise *pooled
// stays null and x holds every row.
int run_bert(mx_encoder *enc, mx_stream *s, float *x, const float *mask, const int32_t *kvl,
             int64_t B, int64_t S, const Rows &rows, float **pooled = nullptr) {
  int rc = bert_pre(enc, s, x, S, rows);
  const size_t L = enc->layers.size();
  const bool prune = pooled && enc->prune_cls && enc->desc.cls_pool;
  for (size_t l = 0; !rc && l < L; ++l) {
    if (!prune || l + 1 < L) {
      rc = bert_layer(enc, s, x, mask, kvl, B, S, rows, l);
      continue;
    }
    rc = layer_attn(enc, s, mask, kvl, B, S, rows, l, 1);  // the first query's context
    float *xc = reinterpret_cast<float *>(enc->work.qkv);
    uint16_t *cc = enc->work.xb;
    if (!rc) {
      Bracket br(enc, s->stream, CAT_OTHER);
      const hipError_t e = mxk::gather_cls(x, enc->work.ctxb, rows.seq_start, B, S,
                                           enc->desc.hidden, xc, cc, s->stream);
      if (e != hipSuccess) rc = hip_fail(e, "CLS row gather");
    }
    if (!rc) rc = layer_rows(enc, s, xc, cc, B, l);
    if (!rc) *pooled = xc;
  }
  return rc;
}

// cls_rows (nullable): when only each sequence's first row of the final
// hidden state is wanted (the ViT head) and CLS pruning is on, the last layer
// computes attention for the first query only and its attention-out, FFN and
// the final LayerNorm over those B rows, gathered into the QKV buffer (free
// once attention has run); *cls_rows points at them (row b for sequence b).
// Otherwise *cls_rows stays null and x holds every row.
int run_preln(mx_encoder *enc, mx_stream *s, float *x, const float *mask, const int32_t *kvl,
              int64_t B, int64_t S, float **cls_rows = nullptr) {
  const int64_t M = B * S, d = enc->desc.hidden, f = enc->desc.ffn;
  const int epi = enc->desc.gelu == MX_GELU_POLY ? MX_EPI_GELU_POLY : MX_EPI_GELU_ERF;
  const size_t L = enc->layers.size();
  const bool prune = cls_rows && enc->prune_cls;
  float *xc = reinterpret_cast<float *>(enc->work.qkv);
  int rc = MX_OK;
  for (size_t l = 0; !rc && l < L; ++l) {
    const LayerW &w = enc->layers[l];
    const bool last = prune && l + 1 == L;
    rc = site_ln(enc, s, x, nullptr, MX_F32, w.ln[0], w.ln[1], M, nullptr, w.ias[SITE_QKV]);
    if (!rc)
      rc = site_gemm(enc, s, w, SITE_QKV, enc->work.xb, M, d, 3 * d, MX_EPI_NONE, nullptr, enc->work.qkv,
                     MX_BF16);
    if (!rc) rc = attn_l(enc, s, B, S, mask, kvl, nullptr, last ? 1 : 0);
    // the rows the rest of the layer runs over
    int64_t Mr = M;
    float *xr = x;
    const uint16_t *ctx = enc->work.ctxb;
    if (!rc && last) {
      Bracket br(enc, s->stream, CAT_OTHER);
      const hipError_t e =
          mxk::gather_cls(x, enc->work.ctxb, nullptr, B, S, d, xc, enc->work.xb, s->stream);
      if (e != hipSuccess) rc = hip_fail(e, "CLS row gather");
      Mr = B;
      xr = xc;
      ctx = enc->work.xb;
    }
    if (!rc && enc->i8) rc = quant_l(enc, s, ctx, MX_BF16, Mr, d, w.ias[SITE_AO]);
    if (!rc) rc = site_gemm(enc, s, w, SITE_AO, ctx, Mr, d, d, MX_EPI_NONE, xr, xr, MX_F32);
    if (!rc) rc = site_ln(enc, s, xr, nullptr, MX_F32, w.ln[2], w.ln[3], Mr, nullptr, w.ias[SITE_UP]);
    // int8: FFN-up's activation in fp32 up to its quantiser, as the dequantise
    // -> GELU -> quantise_a_int8 sequence keeps it (npu_ops.cpp:334-361)
    if (!rc)
      rc = site_gemm(enc, s, w, SITE_UP, enc->work.xb, Mr, d, f, epi, nullptr, enc->work.up,
                     enc->i8 ? MX_F32 : MX_BF16);
    if (!rc && enc->i8) rc = quant_l(enc, s, enc->work.up, MX_F32, Mr, f, w.ias[SITE_DOWN]);
    if (!rc) rc = site_gemm(enc, s, w, SITE_DOWN, enc->work.up, Mr, f, d, MX_EPI_NONE, xr, xr, MX_F32);
  }
  const bool pruned = prune && L > 0;
  float *xf = pruned ? xc : x;
  if (!rc)
    rc = ln_l(enc, s, xf, MX_F32, nullptr, MX_F32, enc->fin_ln[0], enc->fin_ln[1],
              pruned ? B : M, xf, nullptr);
  if (!rc && pruned) *cls_rows = xc;
  return rc;
}

int run_impl(mx_encoder *enc, mx_stream *s, float *x, const float *mask, const int32_t *kvl,
             int64_t B, int64_t S, const Rows *rows = nullptr) {
  const Rows dense{B * S};
  return enc->desc.arch == MX_ARCH_BERT ? run_bert(enc, s, x, mask, kvl, B, S, rows ? *rows : dense)
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

int ensure_front_ws(mx_encoder *enc, mx_stream *s, int64_t B) {
  if (B <= enc->fw_batch) return MX_OK;
  free_dev(enc->f_rows);
  free_dev(enc->f_cls);
  free_dev(enc->f_mel);
  free_dev(enc->f_out1);
  free_dev(enc->f_patch);
  free_dev(enc->f_x);
  enc->fw_batch = 0;
  const mx_encoder_desc &dd = enc->desc;
  const int64_t d = dd.hidden;
  int rc = MX_OK;
  if (dd.front == MX_FRONT_VIT) {
    const int64_t g = dd.image / dd.patch, np = g * g, pd = 3 * dd.patch * dd.patch;
    rc = dev_alloc((void **)&enc->f_rows, B * np * pd * 2, "workspace patch rows");
    if (!rc) rc = dev_alloc((void **)&enc->f_patch, B * np * d * 4, "workspace patch out");
    if (!rc) rc = dev_alloc((void **)&enc->f_x, B * (np + 1) * d * 4, "workspace hidden");
    if (!rc) rc = dev_alloc((void **)&enc->f_cls, B * d * 2, "workspace cls rows");
  } else {
    const int64_t T = dd.frames;
    rc = dev_alloc((void **)&enc->f_mel, B * (T + 2) * dd.mels * 2, "workspace mel");
    if (!rc) rc = dev_alloc((void **)&enc->f_out1, B * (T + 2) * d * 2, "workspace conv1");
    // The conv1 GEMM writes frames 1..T of each sample; the zero frame before
    // and after (conv2's padding) is cleared once here and never written.
    if (!rc) {
      const hipError_t e = hipMemsetAsync(enc->f_out1, 0, B * (T + 2) * d * 2, s->stream);
      if (e != hipSuccess) rc = hip_fail(e, "clearing the conv1 workspace");
    }
  }
  if (rc) return rc;
  enc->fw_batch = B;
  return MX_OK;
}

// The front ends run under the reference's `conv` code: with a placement set,
// it must list conv too (besides the layer's codes).
int check_front_placement() {
  const std::set<std::string> ops = placed_ops();
  if (ops.empty() || ops.count("conv")) return MX_OK;
  return fail(MX_E_INVALID,
              "encoder front end: --npu-ops lists layer ops but not conv, which would keep the "
              "patch/conv front end on the host; the GPU front end runs under conv");
}

int front_gemm(mx_encoder *enc, mx_stream *s, const uint16_t *A, int64_t lda, int64_t M,
               int64_t K, const uint16_t *Wt, int64_t N, const float *bias, int epi,
               const float *resid, void *C, int c_bf16, int64_t ldc) {
  Bracket br(enc, s->stream, CAT_OTHER);
  mxk::GemmArgs a{A, lda, Wt, M, N, K, bias, epi, resid, C, c_bf16, ldc};
  const hipError_t e = mxk::gemm(a, s->stream);
  return e == hipSuccess ? MX_OK : hip_fail(e, "front-end gemm launch");
}

const char *kGemmNames[4] = {"qkv", "attn_out", "ffn_up", "ffn_down"};

// A row-major int8 [K, N] operand -> a new [N, K] device panel.
int stage_i8_panel(mx_ctx *ctx, const int8_t *kn, int64_t K, int64_t N, int8_t **out) {
  if (K % 16)
    return fail(MX_E_INVALID, "int8 operand: K = " + std::to_string(K) +
                                  " is not a multiple of 16");
  std::vector<int8_t> panel(static_cast<size_t>(K) * N);
  for (int64_t k = 0; k < K; ++k)
    for (int64_t n = 0; n < N; ++n)
      panel[static_cast<size_t>(n) * K + k] = kn[static_cast<size_t>(k) * N + n];
  void *p = nullptr;
  hipError_t e = dev_malloc((void **)&p, panel.size());
  if (e == hipSuccess) e = upload(p, panel.data(), panel.size());
  if (e != hipSuccess) {
    if (p) (void)hipFree(p);
    return hip_fail(e, "int8 operand upload");
  }
  *out = static_cast<int8_t *>(p);
  return MX_OK;
}

void free_weights(mx_encoder *enc) {
  for (auto &l : enc->layers) {
    for (auto &p : l.w) free_dev(p);
    for (auto &p : l.b) free_dev(p);
    for (auto &p : l.ln) free_dev(p);
    for (auto &p : l.wq) free_dev(p);
    for (auto &p : l.ws) free_dev(p);
    for (auto &p : l.ias) free_dev(p);
    free_dev(l.wg);
    free_dev(l.wqg);
    free_dev(l.bg);
    free_dev(l.wsg);
  }
  for (auto &p : enc->emb_ln) free_dev(p);
  for (auto &p : enc->fin_ln) free_dev(p);
  free_dev(enc->word);
  free_dev(enc->pos);
  free_dev(enc->type);
  free_dev(enc->patch_w);
  free_dev(enc->head_w);
  free_dev(enc->patch_b);
  free_dev(enc->head_b);
  for (auto &p : enc->conv_w) free_dev(p);
  for (auto &p : enc->conv_b) free_dev(p);
  free_dev(enc->cls_tok);
  free_dev(enc->front_pos);
}

void free_workspace(mx_encoder *enc) {
  free_dev(enc->work.xb);
  free_dev(enc->work.qkv);
  free_dev(enc->work.ctxb);
  free_dev(enc->work.up);
  free_dev(enc->work.proj);
  free_dev(enc->work.emb);
  free_dev(enc->work.xq);
  free_dev(enc->work.sa);
  free_dev(enc->work.glu);
  free_dev(enc->rope_cos);
  free_dev(enc->rope_sin);
  free_dev(enc->work.add_mask);
  free_dev(enc->work.kv_len);
  free_dev(enc->work.seq_start);
  free_dev(enc->work.row_pos);
  free_dev(enc->f_rows);
  free_dev(enc->f_cls);
  free_dev(enc->f_mel);
  free_dev(enc->f_out1);
  free_dev(enc->f_patch);
  free_dev(enc->f_x);
  for (auto ev : enc->events) (void)hipEventDestroy(ev);
  enc->events.clear();
  enc->ev_cat.clear();
  for (auto &ev : enc->ev_all)
    if (ev) {
      (void)hipEventDestroy(ev);
      ev = nullptr;
    }
  enc->ws_rows = enc->ws_batch = enc->ws_mask_rows = enc->fw_batch = 0;
  enc->rope_rows = 0;
}

// The refusal of a weight change on an owner whose clones still borrow them.
int refuse_if_cloned(const mx_encoder *enc, const char *what) {
  int n = 0;
  {
    std::lock_guard<std::mutex> lk(g_clone_mu);
    n = enc->live_clones;
  }
  if (n > 0)
    return fail(MX_E_STATE, std::string(what) + ": " + std::to_string(n) +
                                " lane clone(s) borrow this encoder's weights; destroy them "
                                "before changing the weights");
  return MX_OK;
}

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
  // Geometry may come from a container's config: bound it before anything is
  // sized from it (every product below then fits in 64 bits).
  if (d.layers > 4096 || d.hidden > 65536 || d.heads > 4096 || d.ffn > 1048576 ||
      d.vocab < 0 || d.vocab > (1 << 24) || d.max_pos < 0 || d.max_pos > (1 << 20))
    return fail(MX_E_INVALID, "encoder_create: geometry beyond this backend's bounds "
                              "(layers <= 4096, hidden <= 65536, heads <= 4096, ffn <= 2^20, "
                              "vocab <= 2^24, max_seq_len <= 2^20)");
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
  if (d.front != MX_FRONT_NONE && d.arch != MX_ARCH_PRELN)
    return fail(MX_E_INVALID, "encoder_create: a ViT/Whisper front end needs the pre-LN arch");
  if (d.front == MX_FRONT_VIT &&
      (d.patch <= 0 || d.patch % 8 || d.image <= 0 || d.image % d.patch || d.image % 4 ||
       d.labels <= 0 || d.labels % 4 || (3 * d.patch * d.patch) % 32))
    return fail(MX_E_INVALID, "encoder_create: ViT needs patch % 8 == 0, image % patch == 0, "
                              "image % 4 == 0 and labels % 4 == 0");
  if (d.front == MX_FRONT_WHISPER &&
      (d.mels <= 0 || d.frames <= 0 || d.frames % 2 || (3 * d.mels) % 32 || (3 * d.hidden) % 32))
    return fail(MX_E_INVALID, "encoder_create: Whisper needs even frames and 3*mels, "
                              "3*hidden multiples of 32");
  if (d.front != MX_FRONT_NONE && d.front != MX_FRONT_VIT && d.front != MX_FRONT_WHISPER)
    return fail(MX_E_INVALID, "encoder_create: unknown front end " + std::to_string(d.front));
  if (d.gated_ffn != MX_GATED_NONE && d.gated_ffn != MX_GATED_SILU &&
      d.gated_ffn != MX_GATED_GELU_ERF)
    return fail(MX_E_INVALID, "encoder_create: unknown gated_ffn " + std::to_string(d.gated_ffn));
  if ((d.gated_ffn != MX_GATED_NONE || d.rope) && d.arch != MX_ARCH_BERT)
    return fail(MX_E_UNSUPPORTED, "encoder_create: RoPE and the gated FFN are the BERT-family "
                                  "archs' (nomic, gte); the pre-LN stacks have neither");
  if (d.rope && (d.head_dim % 4))
    return fail(MX_E_UNSUPPORTED, "encoder_create: RoPE needs head_dim % 4 == 0");
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
  // An owner with live clones keeps its weights (the clones read them) until
  // the last clone goes; a clone's destroy may be that moment.
  mx_encoder *orphan = nullptr;
  bool keep_weights = false;
  {
    std::lock_guard<std::mutex> lk(g_clone_mu);
    if (enc->owns_weights && enc->live_clones > 0) {
      enc->orphaned = true;
      keep_weights = true;
    } else if (enc->owner && --enc->owner->live_clones == 0 && enc->owner->orphaned) {
      orphan = enc->owner;
    }
  }
  if (use_device(enc->ctx) == MX_OK) {
    free_workspace(enc);
    if (!keep_weights && enc->owns_weights) free_weights(enc);
  }
  if (!keep_weights) delete enc;
  if (orphan) {
    if (use_device(orphan->ctx) == MX_OK) free_weights(orphan);
    delete orphan;
  }
}

}  // extern "C"

mx_ctx *mx::encoder_ctx(const mx_encoder *enc) { return enc->ctx; }
int64_t mx::encoder_hidden(const mx_encoder *enc) { return enc->desc.hidden; }

extern "C" {

int mx_encoder_clone(mx_encoder *enc, mx_encoder **out) {
  clear_error();
  if (!enc || !out) return fail(MX_E_INVALID, "encoder_clone: null argument");
  *out = nullptr;
  int rc = mx_encoder_ready(enc);
  if (rc) return rc;
  auto *c = new mx_encoder();
  c->ctx = enc->ctx;
  c->desc = enc->desc;
  c->owns_weights = false;
  {
    std::lock_guard<std::mutex> lk(g_clone_mu);
    // A clone of a clone borrows from the same owner.
    c->owner = enc->owns_weights ? enc : enc->owner;
    ++c->owner->live_clones;
  }
  c->layers = enc->layers;
  c->wgen = enc->wgen;
  c->fuse_glu = enc->fuse_glu;
  c->i8 = enc->i8;
  c->rope_inv = enc->rope_inv;
  c->packing = enc->packing;
  c->prune_cls = enc->prune_cls;
  c->narrow_c = enc->narrow_c;
  for (int i = 0; i < 2; ++i) {
    c->emb_ln[i] = enc->emb_ln[i];
    c->fin_ln[i] = enc->fin_ln[i];
    c->conv_w[i] = enc->conv_w[i];
    c->conv_b[i] = enc->conv_b[i];
  }
  c->word = enc->word;
  c->pos = enc->pos;
  c->type = enc->type;
  c->patch_w = enc->patch_w;
  c->head_w = enc->head_w;
  c->patch_b = enc->patch_b;
  c->head_b = enc->head_b;
  c->cls_tok = enc->cls_tok;
  c->front_pos = enc->front_pos;
  // The clone's own device tables (RoPE), so it is ready as the owner is.
  rc = mx_encoder_ready(c);
  if (rc) {
    mx_encoder_destroy(c);
    return rc;
  }
  *out = c;
  return MX_OK;
}

int mx_encoder_set(mx_encoder *enc, const char *name_c, const void *host, int dtype,
                   int64_t count) {
  clear_error();
  if (!enc || !name_c || !host) return fail(MX_E_INVALID, "encoder_set: null argument");
  if (!enc->owns_weights)
    return fail(MX_E_STATE, "encoder_set: a lane clone borrows its parent's weights; set them "
                            "on the parent");
  if (int r = refuse_if_cloned(enc, "encoder_set")) return r;
  ++enc->wgen;
  int rc = use_device(enc->ctx);
  if (rc) return rc;
  const std::string name(name_c);
  const int64_t d = enc->desc.hidden, f = enc->desc.ffn;
  auto put_f32_from = [&](float *&dst, const void *src, int64_t want) -> int {
    free_dev(dst);
    int r = dev_alloc((void **)&dst, want * 4, name.c_str());
    if (r) return r;
    const hipError_t e = upload(dst, src, want * 4);
    return e == hipSuccess ? MX_OK : hip_fail(e, name.c_str());
  };
  auto put_f32 = [&](float *&dst, int64_t want) -> int {
    if (dtype != MX_F32) return fail(MX_E_INVALID, name + ": must be MX_F32");
    if (count != want)
      return fail(MX_E_INVALID, name + ": " + std::to_string(count) + " values, " +
                                    std::to_string(want) + " wanted");
    return put_f32_from(dst, host, want);
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
    const int64_t fu = enc->desc.gated_ffn ? 2 * f : f;
    const int64_t K[4] = {d, d, d, f}, N[4] = {3 * d, d, fu, d};
    for (int i = 0; i < 4; ++i) {
      if (rest == kGemmNames[i]) {
        if (count != K[i] * N[i])
          return fail(MX_E_INVALID, name + ": " + std::to_string(count) + " values, a [" +
                                        std::to_string(K[i]) + ", " + std::to_string(N[i]) +
                                        "] operand wanted");
        if (dtype == MX_I8) {
          // An int8 design's operand: its wscale and asmooth come by their
          // own names; the datapath is chosen by mx_encoder_ready.
          int8_t *panel = nullptr;
          int r = stage_i8_panel(enc->ctx, static_cast<const int8_t *>(host), K[i], N[i], &panel);
          if (r) return r;
          free_dev(w.w[i]);
          free_dev(w.wq[i]);
          w.wq[i] = panel;
          return MX_OK;
        }
        uint16_t *panel = nullptr;
        int r = stage_panel(enc->ctx, host, dtype, K[i], N[i], &panel);
        if (r) return r;
        free_dev(w.w[i]);
        free_dev(w.wq[i]);
        w.w[i] = panel;
        return MX_OK;
      }
      if (rest == std::string(kGemmNames[i]) + ".bias") return put_f32(w.b[i], N[i]);
      if (rest == std::string(kGemmNames[i]) + ".wscale") return put_f32(w.ws[i], N[i]);
      if (rest == std::string(kGemmNames[i]) + ".asmooth") {
        // Kept as its reciprocal, computed once here in fp32 as the reference
        // does per operand (bert_encoder.cpp:764-772).
        if (dtype != MX_F32) return fail(MX_E_INVALID, name + ": must be MX_F32");
        if (count != K[i])
          return fail(MX_E_INVALID, name + ": " + std::to_string(count) + " values, " +
                                        std::to_string(K[i]) + " wanted");
        std::vector<float> ias(static_cast<size_t>(K[i]));
        const float *a = static_cast<const float *>(host);
        for (int64_t k = 0; k < K[i]; ++k) ias[k] = 1.0f / a[k];
        return put_f32_from(w.ias[i], ias.data(), K[i]);
      }
    }
    if (rest == "ln1.weight") return put_f32(w.ln[0], d);
    if (rest == "ln1.bias") return put_f32(w.ln[1], d);
    if (rest == "ln2.weight") return put_f32(w.ln[2], d);
    if (rest == "ln2.bias") return put_f32(w.ln[3], d);
    return fail(MX_E_INVALID, "encoder_set: unknown tensor '" + name + "'");
  }
  if (name == "rope.inv_freq") {
    if (!enc->desc.rope) return fail(MX_E_INVALID, "rope.inv_freq: this encoder has no RoPE");
    if (dtype != MX_F32 || count != enc->desc.head_dim / 2)
      return fail(MX_E_INVALID, "rope.inv_freq: MX_F32 [head_dim/2] wanted");
    const float *v = static_cast<const float *>(host);
    enc->rope_inv.assign(v, v + count);
    free_dev(enc->rope_cos);
    free_dev(enc->rope_sin);
    enc->rope_rows = 0;
    return MX_OK;
  }
  if (name == "embeddings.ln.weight") return put_f32(enc->emb_ln[0], d);
  if (name == "embeddings.ln.bias") return put_f32(enc->emb_ln[1], d);
  // ---- front ends and the ViT head ----
  const int64_t fr = enc->desc.front;
  if (fr == MX_FRONT_VIT) {
    const int64_t pd = 3 * enc->desc.patch * enc->desc.patch;
    const int64_t np1 = (enc->desc.image / enc->desc.patch) * (enc->desc.image / enc->desc.patch) + 1;
    if (name == "patch_embed.weight" || name == "head.weight") {
      const bool head = name == "head.weight";
      const int64_t K = head ? d : pd, N = head ? enc->desc.labels : d;
      if (count != K * N)
        return fail(MX_E_INVALID, name + ": a [" + std::to_string(K) + ", " + std::to_string(N) +
                                      "] operand wanted");
      uint16_t *panel = nullptr;
      int r = stage_panel(enc->ctx, host, dtype, K, N, &panel);
      if (r) return r;
      uint16_t *&dst = head ? enc->head_w : enc->patch_w;
      free_dev(dst);
      dst = panel;
      return MX_OK;
    }
    if (name == "patch_embed.bias") return put_f32(enc->patch_b, d);
    if (name == "head.bias") return put_f32(enc->head_b, enc->desc.labels);
    if (name == "cls_token") return put_f32(enc->cls_tok, d);
    if (name == "position") return put_f32(enc->front_pos, np1 * d);
  }
  if (fr == MX_FRONT_WHISPER) {
    for (int i = 0; i < 2; ++i) {
      const std::string base = i == 0 ? "conv1" : "conv2";
      const int64_t cin = i == 0 ? enc->desc.mels : d;
      if (name == base + ".weight") {
        // Conv1d [hidden, cin, 3] -> GEMM operand [K = 3*cin, N = hidden] with
        // K ordered (tap, channel): the im2col row of frame t is then the three
        // time-major rows t-1, t, t+1 back to back.
        if (count != d * cin * 3)
          return fail(MX_E_INVALID, name + ": a [" + std::to_string(d) + ", " +
                                        std::to_string(cin) + ", 3] tensor wanted");
        if (dtype != MX_F32 && dtype != MX_BF16)
          return fail(MX_E_INVALID, name + ": MX_F32 or MX_BF16");
        const size_t es = dtype == MX_F32 ? 4 : 2;
        std::vector<uint8_t> kn(static_cast<size_t>(3 * cin * d) * es);
        const uint8_t *src = static_cast<const uint8_t *>(host);
        for (int64_t c = 0; c < d; ++c)
          for (int64_t m = 0; m < cin; ++m)
            for (int64_t k = 0; k < 3; ++k)
              std::memcpy(&kn[static_cast<size_t>((k * cin + m) * d + c) * es],
                          &src[static_cast<size_t>((c * cin + m) * 3 + k) * es], es);
        uint16_t *panel = nullptr;
        int r = stage_panel(enc->ctx, kn.data(), dtype, 3 * cin, d, &panel);
        if (r) return r;
        free_dev(enc->conv_w[i]);
        enc->conv_w[i] = panel;
        return MX_OK;
      }
      if (name == base + ".bias") return put_f32(enc->conv_b[i], d);
    }
    if (name == "position") return put_f32(enc->front_pos, enc->desc.frames / 2 * d);
  }
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
    const hipError_t e = upload(enc->type, host, count * 4);
    return e == hipSuccess ? MX_OK : hip_fail(e, name.c_str());
  }
  return fail(MX_E_INVALID, "encoder_set: unknown tensor '" + name + "'");
}

}  // extern "C"

namespace {

// mx_encoder_ready's checks, allocating nothing: every tensor of the path
// set, one datapath (*i8: int8), a RoPE frequency.
int check_ready(const mx_encoder *enc, bool *i8_out) {
  // The datapath is the first operand's: bf16, or int8 (BertEncoder's
  // int8 design set). A stack mixing the two is refused by name.
  const bool i8 = !enc->layers.empty() && enc->layers[0].wq[0] != nullptr;
  for (size_t l = 0; l < enc->layers.size(); ++l) {
    const LayerW &w = enc->layers[l];
    const std::string p = "layer." + std::to_string(l) + ".";
    for (int i = 0; i < 4; ++i) {
      if (!w.w[i] && !w.wq[i])
        return fail(MX_E_STATE, "encoder: " + p + kGemmNames[i] + " was never set");
      if (i8 != (w.wq[i] != nullptr))
        return fail(MX_E_STATE, "encoder: " + p + kGemmNames[i] + " is " +
                                    (i8 ? "bf16" : "int8") + " but layer.0.qkv is " +
                                    (i8 ? "int8" : "bf16") +
                                    "; the stack runs one datapath (repack the container)");
      if (i8 && !w.ws[i])
        return fail(MX_E_STATE, "encoder: " + p + kGemmNames[i] + ".wscale was never set");
      if (i8 && !w.ias[i])
        return fail(MX_E_STATE, "encoder: " + p + kGemmNames[i] + ".asmooth was never set");
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
  if (enc->desc.front == MX_FRONT_VIT) {
    const char *miss = !enc->patch_w ? "patch_embed.weight" : !enc->patch_b ? "patch_embed.bias"
                     : !enc->cls_tok ? "cls_token" : !enc->front_pos ? "position"
                     : !enc->head_w ? "head.weight" : !enc->head_b ? "head.bias" : nullptr;
    if (miss) return fail(MX_E_STATE, std::string("encoder: ") + miss + " was never set");
  }
  if (enc->desc.front == MX_FRONT_WHISPER) {
    const char *miss = !enc->conv_w[0] ? "conv1.weight" : !enc->conv_b[0] ? "conv1.bias"
                     : !enc->conv_w[1] ? "conv2.weight" : !enc->conv_b[1] ? "conv2.bias"
                     : !enc->front_pos ? "position" : nullptr;
    if (miss) return fail(MX_E_STATE, std::string("encoder: ") + miss + " was never set");
  }
  if (enc->desc.rope && enc->rope_inv.empty() && !(enc->desc.rope_theta > 0.0))
    return fail(MX_E_STATE, "encoder: RoPE without a frequency set -- a positive rope_theta or "
                            "rope.inv_freq is needed");
  *i8_out = i8;
  return MX_OK;
}

// Whether everything mx_encoder_ready builds on the device is current for an
// embed of sequence length S, so that the embed allocates nothing: the
// datapath flag, the gated FFN's interleaved operands, the RoPE tables.
int check_prepared(const mx_encoder *enc, int64_t S) {
  bool i8 = false;
  const int rc = check_ready(enc, &i8);
  if (rc) return rc;
  const char *stale = nullptr;
  if (i8 != enc->i8) stale = "the datapath";
  if (!stale && enc->owns_weights && enc->fuse_glu && glu_fusable(enc))
    for (const LayerW &w : enc->layers)
      if (w.glu_gen != enc->wgen) stale = "the gated FFN's interleaved operands";
  if (!stale && enc->desc.rope && enc->rope_rows < S) stale = "the RoPE tables";
  if (stale)
    return fail(MX_E_STATE, std::string("encoder_embed_static: ") + stale +
                                " are not built for this call (it allocates nothing); call "
                                "mx_encoder_ready after the last tensor is set");
  return MX_OK;
}

// The argument checks both embeds share.
int embed_args(const mx_encoder *enc, const mx_stream *s, const int32_t *ids,
               const float *attn_mask, int64_t B, int64_t S, const float *out,
               const char *what) {
  const std::string w = what;
  if (!enc || !s || !ids || !attn_mask || !out) return fail(MX_E_INVALID, w + ": null argument");
  if (B <= 0 || S <= 0) return fail(MX_E_INVALID, w + ": empty batch");
  if (enc->desc.arch != MX_ARCH_BERT)
    return fail(MX_E_INVALID, w + ": the text path is the BERT encoder's");
  if (!enc->word || !enc->pos || !enc->type)
    return fail(MX_E_STATE, w + ": embeddings.word/position/token_type not set");
  if (S > enc->desc.max_pos)
    return fail(MX_E_INVALID, w + ": seq " + std::to_string(S) + " exceeds the " +
                                  std::to_string(enc->desc.max_pos) + " position embeddings");
  return MX_OK;
}

// The static scratch handed out in 256-byte aligned pieces, front to back.
struct Carver {
  uint8_t *base;
  size_t cap;
  size_t used = 0;
  static size_t piece(int64_t bytes) { return (static_cast<size_t>(bytes) + 255) & ~size_t(255); }
  template <typename T>
  T *take(int64_t count) {
    T *p = reinterpret_cast<T *>(base + used);
    used += piece(count * static_cast<int64_t>(sizeof(T)));
    return p;
  }
};

// Bytes of the batch-shaped buffers (mask [B, S], kv_len [B], seq_start and
// the launch order [2B + 1]) and of the row-shaped ones for `rows` rows
// (row_pos and the activations of the HBM layout above), in Carver pieces.
size_t plan_bytes(int64_t B, int64_t S) {
  return Carver::piece(B * S * 4) + Carver::piece(B * 4) + Carver::piece((2 * B + 1) * 4);
}
size_t rows_bytes(const mx_encoder *enc, int64_t rows) {
  const int64_t d = enc->desc.hidden, f = enc->desc.ffn;
  const bool gated = enc->desc.gated_ffn != MX_GATED_NONE;
  size_t n = Carver::piece(rows * 4);                                  // row_pos
  const int64_t ab = wide_acts(enc) ? 4 : 2;  // int8 / narrowed C: up and proj in fp32
  n += 2 * Carver::piece(rows * d * 2) + Carver::piece(rows * d * ab);  // xb ctx proj
  n += Carver::piece(rows * 3 * d * 2);                                 // qkv
  n += Carver::piece(rows * (gated ? 2 * f : f) * ab);                 // up
  if (gated) n += Carver::piece(rows * f * ab);                        // glu
  n += Carver::piece(rows * d * 4);                                    // emb
  if (enc->i8) n += Carver::piece(rows * (d > f ? d : f)) + Carver::piece(rows * 4);
  return n;
}
void carve_plan(Carver &c, int64_t B, int64_t S, Work &w) {
  w.add_mask = c.take<float>(B * S);
  w.kv_len = c.take<int32_t>(B);
  w.seq_start = c.take<int32_t>(2 * B + 1);
}
void carve_rows(const mx_encoder *enc, Carver &c, int64_t rows, Work &w) {
  const int64_t d = enc->desc.hidden, f = enc->desc.ffn;
  const bool gated = enc->desc.gated_ffn != MX_GATED_NONE;
  w.row_pos = c.take<int32_t>(rows);
  w.xb = c.take<uint16_t>(rows * d);
  w.ctxb = c.take<uint16_t>(rows * d);
  const int64_t ab = wide_acts(enc) ? 2 : 1;  // int8 / narrowed C: up and proj in fp32
  w.proj = c.take<uint16_t>(rows * d * ab);
  w.qkv = c.take<uint16_t>(rows * 3 * d);
  w.up = c.take<uint16_t>(rows * (gated ? 2 * f : f) * ab);
  if (gated) w.glu = c.take<uint16_t>(rows * f * ab);
  w.emb = c.take<float>(rows * d);
  if (enc->i8) {
    w.xq = c.take<int8_t>(rows * (d > f ? d : f));
    w.sa = c.take<float>(rows);
  }
}
int scratch_refusal(const mx_encoder *enc, int64_t B, int64_t S, int64_t rows, size_t need,
                    size_t cap, bool packed) {
  return fail(MX_E_INVALID,
              "encoder_embed_static: " + std::to_string(B) + " x " + std::to_string(S) +
                  (packed ? " packs to " + std::to_string(rows) + " rows" : " is " +
                   std::to_string(rows) + " rows") + " of hidden " +
                  std::to_string(enc->desc.hidden) + ", whose workspace needs " +
                  std::to_string(need) + " bytes; the static scratch holds " +
                  std::to_string(cap) + " (MX_STATIC_SCRATCH_BYTES)");
}

// One embed call: its stream, its workspace, its inputs and output rows,
// and -- once its plan is read -- the rows it computes.
struct Pass {
  mx_stream *s = nullptr;
  Work w;
  const int32_t *ids = nullptr;
  const float *mask = nullptr;
  float *out = nullptr;
  int64_t B = 0, S = 0;
  Rows rows{0};
};

// The pass's additive mask, kv_len and plan (seq_start, attention's order).
int pass_plan(mx_encoder *enc, Pass &p) {
  Bracket br(enc, p.s->stream, CAT_OTHER);
  hipError_t e = mxk::mask_build(p.mask, p.B, p.S, p.w.add_mask, p.w.kv_len, p.s->stream);
  // The packed total also goes to the stream's flag block (word 1), read with
  // the refusal flag at the end of the call: the next pass's tile hint.
  if (e == hipSuccess)
    e = mxk::pack_plan(p.w.kv_len, p.B, p.w.seq_start, p.w.seq_start + p.B + 1, p.s->stream,
                       p.s->err_dev + 1);
  return e == hipSuccess ? MX_OK : hip_fail(e, "embed launch");
}

// The pass's rows and its embedding sum. With token packing the launches are
// sized on the host for B * S rows and the packed total stays on the device,
// where every row-wise kernel of the pass reads it (enc->live): the host never
// waits in the middle of the call. Three cases read it back instead: timing
// (the whole plan, for the attention work), the static scratch (carve, which
// takes the row-shaped buffers for exactly that many rows) and the first
// packed pass on a stream (no earlier total to choose the GEMM tiles by).
int pass_rows(mx_encoder *enc, Pass &p, Carver *carve) {
  Bracket br(enc, p.s->stream, CAT_OTHER);
  const int64_t B = p.B, S = p.S;
  int32_t *order = p.w.seq_start + B + 1;
  hipError_t e = hipSuccess;
  p.rows = Rows{B * S};
  if (enc->packing) {
    int64_t total = B * S;
    enc->packed_sq = 0.0;
    if (enc->timing) {
      enc->plan_host.resize(static_cast<size_t>(B + 1));
      e = hipMemcpyAsync(enc->plan_host.data(), p.w.seq_start, (B + 1) * sizeof(int32_t),
                         hipMemcpyDeviceToHost, p.s->stream);
      if (e == hipSuccess) e = hipStreamSynchronize(p.s->stream);
      if (e == hipSuccess) {
        total = enc->plan_host[B];
        for (int64_t b = 0; b < B; ++b) {
          const double L = enc->plan_host[b + 1] - enc->plan_host[b];
          enc->packed_sq += L * L;
        }
      }
    } else if (carve || p.s->last_rows <= 0) {
      // (also the first packed pass on a stream: no earlier total to pick the
      // GEMM tiles by)
      int32_t t = 0;
      e = hipMemcpyAsync(&t, p.w.seq_start + B, sizeof(int32_t), hipMemcpyDeviceToHost,
                         p.s->stream);
      if (e == hipSuccess) e = hipStreamSynchronize(p.s->stream);
      total = t;
      if (e == hipSuccess && t > 0) p.s->last_rows = t;
    } else {
      enc->live = mx::Live{p.w.seq_start + B, p.s->last_rows};
      enc->live_bound = B * S;
    }
    if (e != hipSuccess) return hip_fail(e, "reading the packed row count");
    if (carve) {
      const size_t need = carve->used + rows_bytes(enc, total);
      if (need > carve->cap) return scratch_refusal(enc, B, S, total, need, carve->cap, true);
      carve_rows(enc, *carve, total, p.w);
    }
    e = mxk::embed_sum_packed(p.ids, B, S, enc->desc.hidden, enc->word, enc->desc.vocab,
                              enc->pos, enc->type, p.w.kv_len, p.w.seq_start, p.w.emb,
                              p.w.row_pos, p.s->err_dev, p.s->stream);
    p.rows = Rows{total, p.w.seq_start, p.w.row_pos, order};
  } else {
    e = mxk::embed_sum(p.ids, B, S, enc->desc.hidden, enc->word, enc->desc.vocab, enc->pos,
                       enc->type, p.w.emb, p.s->err_dev, p.s->stream);
    p.rows.order = order;
  }
  return e == hipSuccess ? MX_OK : hip_fail(e, "embed launch");
}

// pooled: the sequences' first rows alone (run_bert's CLS pruning), or null
// for the pass's rows in p.w.emb.
int pass_pool(mx_encoder *enc, Pass &p, const float *pooled) {
  Bracket br(enc, p.s->stream, CAT_OTHER);
  const hipError_t e =
      pooled ? mxk::pool_rows(pooled, p.mask, p.B, p.S, enc->desc.hidden, 1,
                              enc->desc.l2_normalize, p.out, p.s->err_dev, p.s->stream, nullptr,
                              true)
             : mxk::pool_rows(p.w.emb, p.mask, p.B, p.S, enc->desc.hidden, enc->desc.cls_pool,
                              enc->desc.l2_normalize, p.out, p.s->err_dev, p.s->stream,
                              p.rows.seq_start);
  return e == hipSuccess ? MX_OK : hip_fail(e, "pool launch");
}

// The refusals a pass's kernels raise on the data (flag bits of its stream).
int data_refusal(const mx_encoder *enc, int flags) {
  if (flags & 1)
    return fail(MX_E_DATA, "encoder_embed: a token id is outside [0, " +
                               std::to_string(enc->desc.vocab) + ")");
  if (flags & 2) return fail(MX_E_DATA, "CLS pooling on a sequence whose first token is masked");
  return MX_OK;
}

// EmbedService::chunk minus the tokenizer (embed_service.cpp:29-64) over the
// pass: mask and plan, rows and the embedding sum, the stack, pooling, with
// enc->work the pass's workspace while its kernels are launched. carve: the
// static scratch.
int embed_pass(mx_encoder *enc, Pass &p, Carver *carve) {
  int rc = begin_timing(enc, p.s);
  if (!rc) rc = pass_plan(enc, p);
  if (!rc) rc = pass_rows(enc, p, carve);
  enc->work = p.w;
  float *pooled = nullptr;
  if (!rc) rc = run_bert(enc, p.s, p.w.emb, p.w.add_mask, p.w.kv_len, p.B, p.S, p.rows, &pooled);
  if (!rc) rc = pass_pool(enc, p, pooled);
  if (!rc) end_timing(enc, p.s);
  return rc;
}

// mx_encoder_embed; carve: the static scratch instead of the encoder's
// workspace (mx_encoder_embed_static); wait: read the refusal flag at the end
// (synchronising the stream), else leave it for mx_sync
// (mx_encoder_embed_async).
int embed_body(mx_encoder *enc, mx_stream *s, const int32_t *ids, const float *attn_mask,
               int64_t B, int64_t S, float *out, Carver *carve, bool wait = true) {
  Pass p;
  p.s = s;
  p.w = enc->work;
  p.ids = ids;
  p.mask = attn_mask;
  p.out = out;
  p.B = B;
  p.S = S;
  if (carve) {
    const size_t need = plan_bytes(B, S) + (enc->packing ? 0 : rows_bytes(enc, B * S));
    if (need > carve->cap) return scratch_refusal(enc, B, S, B * S, need, carve->cap, false);
    carve_plan(*carve, B, S, p.w);
    if (!enc->packing) carve_rows(enc, *carve, B * S, p.w);
  }
  const Work own = enc->work;
  int rc = embed_pass(enc, p, carve);
  enc->work = own;
  enc->live = mx::Live{};
  enc->live_bound = 0;
  if (rc || !wait) return rc;
  int flags = 0;
  rc = take_data_error(s, &flags);
  return rc ? rc : data_refusal(enc, flags);
}

}  // namespace

extern "C" {

int mx_encoder_ready(mx_encoder *enc) {
  if (!enc) return fail(MX_E_INVALID, "encoder_ready: null encoder");
  bool i8 = false;
  int rc = check_ready(enc, &i8);
  if (rc) return rc;
  enc->i8 = i8;
  rc = ensure_glu_operands(enc);
  // The RoPE tables for every position the text path embeds (S <= max_pos),
  // built here once so that no embed needs to allocate them.
  if (!rc && enc->desc.rope && enc->rope_rows < enc->desc.max_pos) {
    rc = use_device(enc->ctx);
    if (!rc) rc = ensure_rope(enc, enc->desc.max_pos);
  }
  return rc;
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
  int rc = embed_args(enc, s, ids, attn_mask, B, S, out, "encoder_embed");
  if (!rc) rc = use_device(enc->ctx);
  if (!rc) rc = check_placement();
  if (!rc) rc = mx_encoder_ready(enc);
  if (!rc) rc = ensure_ws(enc, B, S);
  if (rc) return rc;
  return embed_body(enc, s, ids, attn_mask, B, S, out, nullptr);
}

int mx_encoder_embed_async(mx_encoder *enc, mx_stream *s, const int32_t *ids,
                           const float *attn_mask, int64_t B, int64_t S, float *out) {
  clear_error();
  int rc = embed_args(enc, s, ids, attn_mask, B, S, out, "encoder_embed_async");
  if (!rc) rc = use_device(enc->ctx);
  if (!rc) rc = check_placement();
  if (!rc) rc = mx_encoder_ready(enc);
  if (!rc) rc = ensure_ws(enc, B, S);
  if (rc) return rc;
  return embed_body(enc, s, ids, attn_mask, B, S, out, nullptr, false);
}

int mx_encoder_embed_static(mx_encoder *enc, mx_stream *s, const int32_t *ids,
                            const float *attn_mask, int64_t B, int64_t S, float *out) {
  clear_error();
  int rc = embed_args(enc, s, ids, attn_mask, B, S, out, "encoder_embed_static");
  if (rc) return rc;
  if (enc->timing)
    return fail(MX_E_STATE, "encoder_embed_static: timing is on (its events are created on "
                            "demand); mx_encoder_set_timing(enc, 0) first");
  // The call reads the packed row count and the refusal flag back with stream
  // synchronisations, which a capturing stream does not allow: refused before
  // any launch or copy.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(s->stream, &cap);
  if (e != hipSuccess) return hip_fail(e, "encoder_embed_static: hipStreamIsCapturing");
  if (cap != hipStreamCaptureStatusNone)
    return fail(MX_E_STATE, "encoder_embed_static: the stream is capturing a graph; this call "
                            "synchronises its stream and cannot be captured");
  void *scratch = nullptr;
  rc = use_device(enc->ctx);
  if (!rc) rc = static_scratch(enc->ctx->device, &scratch);
  if (!rc) rc = check_placement();
  if (!rc) rc = check_prepared(enc, S);
  if (rc) return rc;
  // One call at a time per GPU: the guard is held until the call has
  // synchronised its stream (embed_body ends with that), so the scratch is
  // idle again when it is released.
  const int device = enc->ctx->device;
  rc = static_guard_enter(device, "encoder_embed_static");
  if (rc) return rc;
  Carver carve{static_cast<uint8_t *>(scratch), static_scratch_bytes()};
  const Work own = enc->work;  // the encoder's workspace, back in place on return
  enc->work = Work{};
  rc = embed_body(enc, s, ids, attn_mask, B, S, out, &carve);
  enc->work = own;
  if (rc) {
    // A failed call may leave work queued that uses the scratch: drain the
    // stream before the guard is given back.
    const std::string msg = mx_last_error();
    (void)hipStreamSynchronize(s->stream);
    set_error(msg);
  }
  static_guard_leave(device);
  return rc;
}

int mx_encoder_vit(mx_encoder *enc, mx_stream *s, const float *pixels, int64_t B, float *logits,
                   float *hidden) {
  clear_error();
  if (!enc || !s || !pixels || !logits) return fail(MX_E_INVALID, "encoder_vit: null argument");
  if (enc->desc.front != MX_FRONT_VIT)
    return fail(MX_E_INVALID, "encoder_vit: this encoder was created without the ViT front end");
  if (B <= 0) return fail(MX_E_INVALID, "encoder_vit: empty batch");
  const mx_encoder_desc &dd = enc->desc;
  const int64_t d = dd.hidden, g = dd.image / dd.patch, np = g * g, S = np + 1;
  const int64_t pd = 3 * dd.patch * dd.patch;
  int rc = use_device(enc->ctx);
  if (!rc) rc = check_placement();
  if (!rc) rc = check_front_placement();
  if (!rc) rc = mx_encoder_ready(enc);
  if (!rc) rc = ensure_ws(enc, B, S);
  if (!rc) rc = ensure_front_ws(enc, s, B);
  if (!rc) rc = begin_timing(enc, s);
  if (rc) return rc;
  float *x = hidden ? hidden : enc->f_x;
  {
    Bracket br(enc, s->stream, CAT_OTHER);
    const hipError_t e = mxk::vit_patches(pixels, B, (int)dd.image, (int)dd.patch, enc->f_rows,
                                          s->stream);
    if (e != hipSuccess) return hip_fail(e, "vit patches launch");
  }
  rc = front_gemm(enc, s, enc->f_rows, pd, B * np, pd, enc->patch_w, d, enc->patch_b,
                  MX_EPI_NONE, nullptr, enc->f_patch, 0, d);
  if (rc) return rc;
  {
    Bracket br(enc, s->stream, CAT_OTHER);
    const hipError_t e = mxk::vit_assemble(enc->f_patch, enc->cls_tok, enc->front_pos, B,
                                           (int)np, (int)d, x, s->stream);
    if (e != hipSuccess) return hip_fail(e, "vit assemble launch");
  }
  // Without a hidden state to return, only the CLS rows reach the head.
  float *cls_rows = nullptr;
  rc = run_preln(enc, s, x, nullptr, nullptr, B, S, hidden ? nullptr : &cls_rows);
  if (rc) return rc;
  {
    Bracket br(enc, s->stream, CAT_OTHER);
    const hipError_t e =
        cls_rows ? mxk::gather_rows_bf16(cls_rows, d, B, (int)d, enc->f_cls, s->stream)
                 : mxk::gather_rows_bf16(x, S * d, B, (int)d, enc->f_cls, s->stream);
    if (e != hipSuccess) return hip_fail(e, "cls gather launch");
  }
  rc = front_gemm(enc, s, enc->f_cls, d, B, d, enc->head_w, dd.labels, enc->head_b, MX_EPI_NONE,
                  nullptr, logits, 0, dd.labels);
  if (rc) return rc;
  end_timing(enc, s);
  return mx_sync(s);
}

int mx_encoder_whisper(mx_encoder *enc, mx_stream *s, const float *mel, int64_t B,
                       float *hidden) {
  clear_error();
  if (!enc || !s || !mel || !hidden) return fail(MX_E_INVALID, "encoder_whisper: null argument");
  if (enc->desc.front != MX_FRONT_WHISPER)
    return fail(MX_E_INVALID,
                "encoder_whisper: this encoder was created without the Whisper front end");
  if (B <= 0) return fail(MX_E_INVALID, "encoder_whisper: empty batch");
  const mx_encoder_desc &dd = enc->desc;
  const int64_t d = dd.hidden, T = dd.frames, S = T / 2, cin = dd.mels;
  int rc = use_device(enc->ctx);
  if (!rc) rc = check_placement();
  if (!rc) rc = check_front_placement();
  if (!rc) rc = mx_encoder_ready(enc);
  if (!rc) rc = ensure_ws(enc, B, S);
  if (!rc) rc = ensure_front_ws(enc, s, B);
  if (!rc) rc = begin_timing(enc, s);
  if (rc) return rc;
  {
    Bracket br(enc, s->stream, CAT_OTHER);
    const hipError_t e = mxk::mel_time_major(mel, B, (int)cin, (int)T, enc->f_mel, s->stream);
    if (e != hipSuccess) return hip_fail(e, "mel transpose launch");
  }
  for (int64_t b = 0; !rc && b < B; ++b) {
    // conv1: the im2col row of frame t is time-major rows t..t+2 of the padded
    // copy, i.e. row stride mels and K = 3 * mels (overlapping rows).
    rc = front_gemm(enc, s, enc->f_mel + b * (T + 2) * cin, cin, T, 3 * cin, enc->conv_w[0], d,
                    enc->conv_b[0], MX_EPI_GELU_ERF, nullptr,
                    enc->f_out1 + (b * (T + 2) + 1) * d, 1, d);
    // conv2 (stride 2): output frame u reads padded rows 2u..2u+2, row stride
    // 2 * hidden, K = 3 * hidden; the positions enter as the fused residual.
    if (!rc)
      rc = front_gemm(enc, s, enc->f_out1 + b * (T + 2) * d, 2 * d, S, 3 * d, enc->conv_w[1], d,
                      enc->conv_b[1], MX_EPI_GELU_ERF, enc->front_pos, hidden + b * S * d, 0, d);
  }
  if (!rc) rc = run_preln(enc, s, hidden, nullptr, nullptr, B, S);
  if (rc) return rc;
  end_timing(enc, s);
  return mx_sync(s);
}

int mx_encoder_set_packing(mx_encoder *enc, int on) {
  clear_error();
  if (!enc) return fail(MX_E_INVALID, "encoder_set_packing: null encoder");
  enc->packing = on != 0;
  return MX_OK;
}

int mx_encoder_set_cls_pruning(mx_encoder *enc, int on) {
  clear_error();
  if (!enc) return fail(MX_E_INVALID, "encoder_set_cls_pruning: null encoder");
  enc->prune_cls = on != 0;
  return MX_OK;
}

int mx_encoder_set_fusion(mx_encoder *enc, int on) {
  clear_error();
  if (!enc) return fail(MX_E_INVALID, "encoder_set_fusion: null encoder");
  enc->fuse_glu = on != 0;
  return MX_OK;
}

int mx_encoder_set_narrowed_c(mx_encoder *enc, int on) {
  clear_error();
  if (!enc) return fail(MX_E_INVALID, "encoder_set_narrowed_c: null encoder");
  if (on && (enc->desc.arch != MX_ARCH_BERT || enc->desc.front != MX_FRONT_NONE))
    return fail(MX_E_UNSUPPORTED, "encoder_set_narrowed_c: the narrowed C is the BERT stack's "
                                  "datapath (bert_encoder.cpp:741-924); the pre-LN encoders add "
                                  "their projections into the residual in the GEMM epilogue");
  enc->narrow_c = on != 0;
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

// A pre-tiled container operand by its container name: the layer GEMMs, and
// the ViT patch embedding and head.
int mx_encoder_set_panel(mx_encoder *enc, const char *name_c, const uint16_t *panel, int64_t K,
                         int64_t N, int64_t tile_k, int64_t tile_n, int64_t mac_s,
                         int64_t mac_t) {
  clear_error();
  if (!enc || !name_c || !panel) return fail(MX_E_INVALID, "encoder_set_panel: null argument");
  if (!enc->owns_weights)
    return fail(MX_E_STATE, "encoder_set_panel: a lane clone borrows its parent's weights");
  if (int r = refuse_if_cloned(enc, "encoder_set_panel")) return r;
  ++enc->wgen;
  const std::string name(name_c);
  const int64_t d = enc->desc.hidden, f = enc->desc.ffn;
  uint16_t **dst = nullptr;
  int64_t wantK = 0, wantN = 0;
  if (name.rfind("layer.", 0) == 0) {
    size_t p = 6;
    int64_t L = 0;
    bool digits = false;
    while (p < name.size() && std::isdigit(static_cast<unsigned char>(name[p]))) {
      L = L * 10 + (name[p] - '0');
      ++p;
      digits = true;
    }
    if (digits && p < name.size() && name[p] == '.' && L < enc->desc.layers) {
      const std::string rest = name.substr(p + 1);
      const int64_t Ks[4] = {d, d, d, f};
      const int64_t Ns[4] = {3 * d, d, enc->desc.gated_ffn ? 2 * f : f, d};
      for (int i = 0; i < 4; ++i)
        if (rest == kGemmNames[i]) {
          dst = &enc->layers[static_cast<size_t>(L)].w[i];
          wantK = Ks[i];
          wantN = Ns[i];
        }
    }
  } else if (enc->desc.front == MX_FRONT_VIT && name == "patch_embed.weight") {
    dst = &enc->patch_w;
    wantK = 3 * enc->desc.patch * enc->desc.patch;
    wantN = d;
  } else if (enc->desc.front == MX_FRONT_VIT && name == "head.weight") {
    dst = &enc->head_w;
    wantK = d;
    wantN = enc->desc.labels;
  }
  if (!dst) return fail(MX_E_INVALID, "encoder_set_panel: '" + name + "' is not a GEMM operand "
                                      "of this encoder");
  if (K != wantK || N != wantN)
    return fail(MX_E_INVALID, name + ": a [" + std::to_string(K) + ", " + std::to_string(N) +
                                  "] panel, a [" + std::to_string(wantK) + ", " +
                                  std::to_string(wantN) + "] operand wanted");
  uint16_t *wt = nullptr;
  const int rc = stage_tiled_panel(enc->ctx, panel, K, N, tile_k, tile_n, mac_s, mac_t, &wt);
  if (rc) return rc;
  free_dev(*dst);
  *dst = wt;
  return MX_OK;
}

int mx_encoder_from_npue(mx_ctx *ctx, const mx_npue *f, mx_encoder **out) {
  clear_error();
  if (!ctx || !f || !out) return fail(MX_E_INVALID, "encoder_from_npue: null argument");
  *out = nullptr;
  auto cfg = [&](const char *key, std::string &v) -> int {
    if (!npue_config(f, key, v)) return fail(MX_E_INVALID, std::string(".npue: no config key ") + key);
    return MX_OK;
  };
  auto cfg_int = [&](const char *key, int64_t &v) -> int {
    std::string t;
    int rc = cfg(key, t);
    if (rc) return rc;
    char *end = nullptr;
    v = std::strtoll(t.c_str(), &end, 10);
    if (t.empty() || *end)
      return fail(MX_E_INVALID, std::string(".npue: config ") + key + " = '" + t +
                                    "' is not an integer");
    return MX_OK;
  };
  std::string arch;
  int rc = cfg("arch", arch);
  if (rc) return rc;
  // The whitelist of app::encoder_implemented (app_state.hpp:175-200), cut to
  // what this backend's stack computes: the post-LN BERT and its RoPE /
  // gated-FFN variants. Each variant's keys are checked as set_model_shape
  // checks them (app_state.hpp:440-550), so a container that leaves the
  // fusion order or the frequencies to guesswork is refused, not guessed.
  const bool nomic = arch == "nomic_bert_rope_swiglu", gte = arch == "gte_new_rope_geglu";
  if (arch != "bert_abs_gelu_postln" && !nomic && !gte)
    return fail(MX_E_UNSUPPORTED,
                ".npue: container arch '" + arch + "' -- this loader builds the post-LN BERT "
                "stack (bert_abs_gelu_postln) and its RoPE/gated-FFN variants "
                "(nomic_bert_rope_swiglu, gte_new_rope_geglu); other archs share its tensor "
                "names but not its maths, and are refused rather than run as BERT");
  int gated = MX_GATED_NONE;
  double rope_theta = 0.0;
  std::vector<float> inv_freq;
  std::string v;
  if (npue_config(f, "gated_ffn", v) && v == "true") gated = MX_GATED_SILU;
  if (nomic || gte) {
    if (!npue_config(f, "position_embedding_type", v) || v != "rope")
      return fail(MX_E_INVALID, ".npue: container arch is " + arch + " but "
                                "position_embedding_type is not 'rope' -- refusing rather than "
                                "guessing how position is encoded");
    if (gated == MX_GATED_NONE)
      return fail(MX_E_INVALID, ".npue: container arch is " + arch + " but gated_ffn is not "
                                "true -- refusing rather than running a plain FFN over a fused "
                                "up|gate weight");
    if (nomic) {
      if (!npue_config(f, "swiglu_halves", v) || v != "fc11_up|fc12_gate")
        return fail(MX_E_INVALID, ".npue: unrecognised swiglu_halves ordering -- expected "
                                  "'fc11_up|fc12_gate'; refusing rather than guessing which half "
                                  "of the fused ffn_up gets SiLU");
      if (!npue_config(f, "rope_theta", v) || !((rope_theta = std::strtod(v.c_str(), nullptr)) > 0))
        return fail(MX_E_INVALID, ".npue: nomic_bert_rope_swiglu container has a non-positive "
                                  "rope_theta");
    } else {
      if (!npue_config(f, "glu_halves", v) || v.rfind("up_first|gate_second", 0) != 0)
        return fail(MX_E_INVALID, ".npue: unrecognised glu_halves ordering -- expected it to "
                                  "begin 'up_first|gate_second'; refusing rather than guessing "
                                  "which half of the fused ffn_up gets the activation");
      if (!npue_config(f, "rope_inv_freq", v))
        return fail(MX_E_INVALID, ".npue: gte_new_rope_geglu container carries no "
                                  "'rope_inv_freq' -- the frequency set is not derivable from "
                                  "rope_theta, so refusing rather than falling back");
      // A JSON array of numbers.
      const char *p = v.c_str();
      while (*p && *p != '[') ++p;
      if (*p == '[') ++p;
      for (;;) {
        while (*p == ' ' || *p == ',' || *p == '\n' || *p == '\t') ++p;
        if (*p == ']' || !*p) break;
        char *e = nullptr;
        const double x = std::strtod(p, &e);
        if (e == p) return fail(MX_E_INVALID, ".npue: rope_inv_freq is not an array of numbers");
        inv_freq.push_back(static_cast<float>(x));
        p = e;
      }
    }
  }
  // The gated activation is read for every gated container, whatever its
  // arch (set_model_shape, app_state.hpp:534-553): a missing key means SiLU
  // except on gte, whose containers must carry it; an unknown value refuses.
  if (gated != MX_GATED_NONE) {
    std::string act;
    if (!npue_config(f, "activation", act)) {
      if (gte)
        return fail(MX_E_INVALID, ".npue: gte_new_rope_geglu container carries no "
                                  "'activation' key -- refusing rather than guessing which "
                                  "activation the gate half gets");
      act = "silu";
    }
    if (act == "silu") gated = MX_GATED_SILU;
    else if (act == "gelu") gated = MX_GATED_GELU_ERF;
    else
      return fail(MX_E_INVALID, ".npue: unknown gated-FFN activation '" + act + "' -- this "
                                "build implements 'silu' and 'gelu' (exact erf)");
  }
  mx_encoder_desc d{};
  d.arch = MX_ARCH_BERT;
  if ((rc = cfg_int("num_layers", d.layers)) || (rc = cfg_int("hidden", d.hidden)) ||
      (rc = cfg_int("num_heads", d.heads)) || (rc = cfg_int("head_dim", d.head_dim)) ||
      (rc = cfg_int("intermediate", d.ffn)) || (rc = cfg_int("max_seq_len", d.max_pos)))
    return rc;
  std::string pool;
  if ((rc = cfg("pooling", pool))) return rc;
  if (pool == "cls") d.cls_pool = 1;
  else if (pool == "mean") d.cls_pool = 0;
  else
    return fail(MX_E_INVALID, ".npue: unknown pooling mode '" + pool + "' -- expected mean or cls");
  std::string l2;
  d.l2_normalize = npue_config(f, "l2_normalize", l2) ? (l2 == "true" ? 1 : 0) : 1;
  std::string layout;
  if (npue_config(f, "gemm_layout", layout) && layout == "host")
    return fail(MX_E_UNSUPPORTED,
                ".npue: this container is gemm_layout \"host\" -- its GEMM operands are "
                "row-major F32 for the CPU, and the GPU GEMM multiplies bf16; repack with bf16 "
                "operands (the reference refuses --npu-ops gemm on such a container too)");
  d.ln_eps = 1e-12f;
  d.attn_scale = 1.0f;  // 1/sqrt(head_dim) is folded into the packed Q block
  d.gelu = MX_GELU_POLY;
  d.gated_ffn = gated;
  d.rope = nomic || gte;
  d.rope_theta = rope_theta;
  if (gte && static_cast<int64_t>(inv_freq.size()) * 2 != d.head_dim)
    return fail(MX_E_INVALID, ".npue: rope_inv_freq has " + std::to_string(inv_freq.size()) +
                                  " entries, expected head_dim/2 = " +
                                  std::to_string(d.head_dim / 2));
  const TensorRecView word = npue_tensor(f, "embeddings.word");
  if (!word.found || word.padded.size() != 2)
    return fail(MX_E_INVALID, ".npue: embeddings.word missing or not [vocab, hidden]");
  d.vocab = word.padded[0];
  mx_encoder *enc = nullptr;
  if ((rc = mx_encoder_create(ctx, &d, &enc))) return rc;
  auto refuse = [&](int code) {
    const std::string msg = mx_last_error();
    mx_encoder_destroy(enc);
    return fail(code, msg);
  };
  auto set_f32 = [&](const std::string &name) -> int {
    const TensorRecView t = npue_tensor(f, name);
    if (!t.found) return fail(MX_E_INVALID, ".npue: no tensor named " + name);
    if (t.dtype != "F32")
      return fail(MX_E_INVALID, name + ": " + t.dtype + " in the container, F32 wanted");
    return mx_encoder_set(enc, name.c_str(), t.data, MX_F32, static_cast<int64_t>(t.nbytes / 4));
  };
  std::vector<std::string> names = {"embeddings.word", "embeddings.position",
                                    "embeddings.token_type", "embeddings.ln.weight",
                                    "embeddings.ln.bias"};
  for (int64_t L = 0; L < d.layers; ++L) {
    const std::string p = "layer." + std::to_string(L) + ".";
    for (int i = 0; i < 4; ++i) names.push_back(p + kGemmNames[i] + ".bias");
    for (const char *n : {"ln1.weight", "ln1.bias", "ln2.weight", "ln2.bias"})
      names.push_back(p + n);
  }
  for (const std::string &n : names)
    if ((rc = set_f32(n))) return refuse(rc);
  if (!inv_freq.empty() &&
      (rc = mx_encoder_set(enc, "rope.inv_freq", inv_freq.data(), MX_F32,
                           static_cast<int64_t>(inv_freq.size()))))
    return refuse(rc);
  for (int64_t L = 0; L < d.layers; ++L)
    for (int i = 0; i < 4; ++i) {
      const std::string n = "layer." + std::to_string(L) + "." + kGemmNames[i];
      const TensorRecView t = npue_tensor(f, n);
      if (!t.found) return refuse(fail(MX_E_INVALID, ".npue: no tensor named " + n));
      if (t.padded.size() != 2)
        return refuse(fail(MX_E_INVALID, n + ": GEMM operand is not two-dimensional"));
      // Shapes come from the file: bound them before any product is formed.
      if (t.padded[0] <= 0 || t.padded[1] <= 0 || t.padded[0] > (1 << 20) ||
          t.padded[1] > (1 << 20))
        return refuse(fail(MX_E_INVALID, n + ": a [" + std::to_string(t.padded[0]) + "," +
                                             std::to_string(t.padded[1]) + "] GEMM operand; "
                                             "each dimension must lie in [1, 2^20]"));
      if (!t.logical.empty() && t.logical != t.padded)
        return refuse(fail(MX_E_INVALID, n + ": logical and padded shapes differ; the GEMM "
                                             "needs them equal (repack)"));
      // I4 is storage over the int8 datapath (common/int4_panel.hpp): the
      // nibbles are widened to the int8 panel on the GPU, then staged as I8.
      const bool i4 = t.dtype == "I4";
      const bool i8 = t.dtype == "I8" || i4;
      if ((t.dtype != "BF16" && !i8) || !t.block_panel)
        return refuse(fail(MX_E_INVALID, n + ": " + t.dtype + " without a block_panel "
                                             "layout; a pre-tiled BF16, I8 or I4 operand is "
                                             "wanted"));
      const int64_t K = t.padded[0], N = t.padded[1];
      if (i4 && (K * N) % 2)
        return refuse(fail(MX_E_INVALID, n + ": I4 payload of [" + std::to_string(K) + "," +
                                             std::to_string(N) + "] holds an odd number of "
                                             "nibbles; two int4 values make a byte"));
      const uint64_t want = static_cast<uint64_t>(i4 ? K * N / 2 : K * N * (i8 ? 1 : 2));
      if (t.nbytes != want)
        return refuse(fail(MX_E_INVALID, n + ": " + std::to_string(t.nbytes) + " bytes for a [" +
                                             std::to_string(K) + "," + std::to_string(N) +
                                             "] " + (i4 ? "int4" : i8 ? "int8" : "bf16") +
                                             " operand (" + std::to_string(want) + " wanted)"));
      if (!i8) {
        rc = mx_encoder_set_panel(enc, n.c_str(), static_cast<const uint16_t *>(t.data), K, N,
                                  t.tile_k, t.tile_n, t.mac_s, t.mac_t);
        if (rc) return refuse(rc);
        continue;
      }
      // An int8 design's operand (tools/lib/gemm_i8.py's scheme; gemm_i4.py's
      // for I4): the panel, its per-column .wscale and per-row .asmooth, all
      // from the mapping.
      const TensorRecView ws = npue_tensor(f, n + ".wscale");
      const TensorRecView sm = npue_tensor(f, n + ".asmooth");
      if (!ws.found || !sm.found)
        return refuse(fail(MX_E_INVALID, n + ": an " + t.dtype + " operand without its " +
                                             (ws.found ? ".asmooth" : ".wscale") +
                                             " -- the container is not a complete int8 pack"));
      if (ws.dtype != "F32" || sm.dtype != "F32" || ws.nbytes != static_cast<uint64_t>(N * 4) ||
          sm.nbytes != static_cast<uint64_t>(K * 4))
        return refuse(fail(MX_E_INVALID, n + ": .wscale must be F32 [" + std::to_string(N) +
                                             "] and .asmooth F32 [" + std::to_string(K) + "]"));
      I8Operand op;
      if (i4) {
        // The group size is config, checked against the sidecar's height
        // (int4_panel.hpp:127-173).
        std::string gtext;
        if (!npue_config(f, "int4_group", gtext))
          return refuse(fail(MX_E_INVALID, n + ": I4 payload, but the container states no "
                                               "int4_group -- the group size says which rows "
                                               "of K share a scale"));
        int64_t group = 0;
        if ((rc = cfg_int("int4_group", group))) return refuse(rc);
        if (group < 0)
          return refuse(fail(MX_E_INVALID, n + ": config int4_group is " +
                                               std::to_string(group) + "; rows per group must "
                                               "be >= 0, where 0 means one group over the "
                                               "whole K"));
        const int64_t g = group == 0 ? K : group, G = (K + g - 1) / g;
        const TensorRecView gs = npue_tensor(f, n + ".gscale");
        if (!gs.found)
          return refuse(fail(MX_E_INVALID, n + ": I4 payload but no " + n + ".gscale in the "
                                               "container -- the group scale is the only thing "
                                               "that puts a nibble back in units of .wscale"));
        if (gs.dtype != "F32" || gs.padded.size() != 2 || gs.padded[0] != G ||
            gs.padded[1] != N || gs.nbytes != static_cast<uint64_t>(G * N * 4))
          return refuse(fail(MX_E_INVALID, n + ".gscale is " + gs.dtype + " with " +
                                               std::to_string(gs.nbytes) + " bytes but "
                                               "int4_group=" + std::to_string(group) +
                                               " over K=" + std::to_string(K) + " needs F32 [" +
                                               std::to_string(G) + "," + std::to_string(N) +
                                               "]"));
        rc = stage_i4(ctx, static_cast<const uint8_t *>(t.data),
                      static_cast<const float *>(gs.data), group,
                      static_cast<const float *>(ws.data), static_cast<const float *>(sm.data), K,
                      N, t.tile_k, t.tile_n, t.mac_s, t.mac_t, &op);
      } else {
        rc = stage_i8(ctx, static_cast<const int8_t *>(t.data),
                      static_cast<const float *>(ws.data), static_cast<const float *>(sm.data), K,
                      N, t.tile_k, t.tile_n, t.mac_s, t.mac_t, &op);
      }
      if (rc) return refuse(rc);
      const int64_t d = enc->desc.hidden, fw = enc->desc.ffn;
      const int64_t Ks[4] = {d, d, d, fw}, Ns[4] = {3 * d, d, gated ? 2 * fw : fw, d};
      if (K != Ks[i] || N != Ns[i]) {
        free_i8(op);
        return refuse(fail(MX_E_INVALID, n + ": a [" + std::to_string(K) + ", " +
                                             std::to_string(N) + "] operand, a [" +
                                             std::to_string(Ks[i]) + ", " +
                                             std::to_string(Ns[i]) + "] one wanted"));
      }
      LayerW &w = enc->layers[static_cast<size_t>(L)];
      ++enc->wgen;
      free_dev(w.w[i]);
      free_dev(w.wq[i]);
      free_dev(w.ws[i]);
      free_dev(w.ias[i]);
      w.wq[i] = op.wq;
      w.ws[i] = op.wscale;
      w.ias[i] = op.ias;
    }
  if ((rc = mx_encoder_ready(enc))) return refuse(rc);
  *out = enc;
  return MX_OK;
}

}  // extern "C"
