// C ABI of libattnnn.so: context, buffer layouts, weight packing and the
// orchestration of a forward (prefill / decode step) over the gfx950 kernels.
//
// One forward over M token rows (B sequences x T tokens):
//   embed_rms                        x = x0 = rms(embed[tok])
//   per layer l:
//     proj  RMS -> qkv^T   STORE     qkv = bf16(rms(x) @ [Wq Wk Wv] * sa0)
//     qkv_post                       q = rope(rms(q)); K/V cache += rope(rms(k)), v
//     attention (+ combine)          window / full-causal, fp32 softmax
//     proj  o^T            RESID_ATTN   x = r0 x + p0 (a @ Wo*sa1) + x0l x0
//     proj  RMS -> fc^T    RELU2     h = relu(rms(x) @ fc)^2
//     proj  proj^T         RESID_MLP x = r1 x + p1 (h @ proj)
//   proj RMS -> lm_head^T  LOGITS    z = bf16(rms(x) @ lm_head) (last rows)
//   sample                           one token per sequence
// `proj` is the GEMV (M <= 8) or the MFMA GEMM.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <string>
#include <vector>
#include "attnnn.h"
#include "launch.h"

using namespace ann;

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define HIPCHK(expr)                                                                  \
  do {                                                                                \
    hipError_t e_ = (expr);                                                           \
    if (e_ != hipSuccess)                                                             \
      return fail(ANN_E_HIP, "%s failed: %s", #expr, hipGetErrorString(e_));          \
  } while (0)

constexpr size_t ALIGN = 256;
constexpr int MAX_SPLIT = AD_MAX_SPLIT;

size_t up(size_t v) { return (v + ALIGN - 1) / ALIGN * ALIGN; }

struct WLayout {  // byte offsets into the packed weight buffer
  size_t embed, head, layer0, layer_stride, qkv, o, fc, proj, lam, cs, sn, total;
};

WLayout weight_layout(const ann_config& c) {
  const size_t d = c.d, V = c.V, Dh = d / c.H;
  WLayout w{};
  size_t off = 0;
  w.embed = off; off += up(V * d * 2);
  w.head = off; off += up(V * d * 2);
  w.qkv = 0;
  w.o = up(3 * d * d * 2);
  w.fc = w.o + up(d * d * 2);
  w.proj = w.fc + up(4 * d * d * 2);
  w.layer_stride = w.proj + up(4 * d * d * 2);
  w.layer0 = off; off += w.layer_stride * c.L;
  w.lam = off; off += up((size_t)c.L * 8 * 4);
  w.cs = off; off += up((size_t)c.max_ctx * (Dh / 4) * 4);
  w.sn = off; off += up((size_t)c.max_ctx * (Dh / 4) * 4);
  w.total = off;
  return w;
}

struct SLayout {  // byte offsets into the workspace
  size_t pos, sp, steps, amax, acnt, pfsink, x, x0, qkv, q, ao, hn, hid, part, zb, pcand, pd,
      qat,
      pd_bytes,
      ce, ce_tz, ce_rows, ce_mean, total;
};

size_t pd_layout(const ann_config& c, int which) {
  return ann::pd_layout((size_t)c.d, (size_t)c.H, which);
}

// 128-column tiles of the lm_head GEMM (its work-group tile width).
int ce_tiles(const ann_config& c) { return (c.V + 127) / 128; }

SLayout ws_layout(const ann_config& c) {
  const size_t d = c.d, M = c.max_tokens, B = c.max_batch, Dh = d / c.H;
  SLayout s{};
  size_t off = 0;
  s.pos = off; off += up(B * 4);
  s.sp = off; off += up(sizeof(SampParams));
  s.steps = off; off += up(B * 8);
  s.amax = off; off += up((B <= 8 ? B : 1) * (size_t)gemv_blocks(c.V, c.d) * 8);
  s.acnt = off; off += up(B * c.H * 4);
  s.pfsink = off; off += up(8);
  s.qat = off; off += up((size_t)c.max_batch * 3 * c.d / 2 * 8);   // fused qkv -> attention words
  s.x = off; off += up(M * d * 2);
  s.x0 = off; off += up(M * d * 2);
  s.qkv = off; off += up(M * 3 * d * 2);
  s.q = off; off += up(M * d * 2);
  s.ao = off; off += up(M * d * 2);
  s.hn = off; off += up(M * d * 2);
  s.hid = off; off += up(M * 4 * d * 2);
  s.part = off; off += up(B * c.H * MAX_SPLIT * (Dh + 1) * 8);
  s.zb = off; off += up(B * (size_t)c.V * 2);
  s.pd = off; off += (s.pd_bytes = up(pd_layout(c, 0)));
  // training-forward loss: per-(128-column tile, row) partial sums, target
  // logits, per-row losses, the mean
  s.ce = off; off += up((size_t)ce_tiles(c) * M * 4);
  s.ce_tz = off; off += up(M * 4);
  s.ce_rows = off; off += up(M * 4);
  s.ce_mean = off; off += up(4);
  // the persistent step's top-k candidates (sampled rows)
  s.pcand = off; off += up((size_t)PD_MAX_B * PD_MAX_G * (TK_M + 1) * 4);
  s.total = off;
  return s;
}

size_t kv_layer_bytes(const ann_config& c) {
  return (size_t)c.max_batch * c.max_ctx * c.d * 2;  // B x H x ctx x Dh bf16
}

int check_config(const ann_config* c) {
  if (!c) return fail(ANN_E_ARG, "config is null");
  if (c->d <= 0 || c->L <= 0 || c->H <= 0 || c->V <= 0)
    return fail(ANN_E_ARG, "d, L, H, V must be positive");
  if (c->d % c->H) return fail(ANN_E_ARG, "d=%d not divisible by H=%d", c->d, c->H);
  const int Dh = c->d / c->H;
  if (Dh != 64 && Dh != 128) return fail(ANN_E_ARG, "head_dim %d unsupported (64 or 128)", Dh);
  if (c->d % 64) return fail(ANN_E_ARG, "d=%d must be a multiple of 64", c->d);
  if (c->V_sample <= 0 || c->V_sample > c->V)
    return fail(ANN_E_ARG, "V_sample=%d outside [1, V=%d]", c->V_sample, c->V);
  if (c->window <= 0) return fail(ANN_E_ARG, "window must be positive");
  if (c->n_long < 0 || c->n_long > ANN_MAX_LONG_LAYERS)
    return fail(ANN_E_ARG, "n_long=%d outside [0, %d]", c->n_long, ANN_MAX_LONG_LAYERS);
  for (int i = 0; i < c->n_long; ++i)
    if (c->long_layers[i] < 0 || c->long_layers[i] >= c->L)
      return fail(ANN_E_ARG, "long layer %d outside [0, %d)", c->long_layers[i], c->L);
  if (c->max_batch <= 0 || c->max_ctx <= 0 || c->max_tokens <= 0)
    return fail(ANN_E_ARG, "max_batch, max_ctx, max_tokens must be positive");
  if (c->max_tokens < c->max_batch)
    return fail(ANN_E_ARG, "max_tokens=%d < max_batch=%d", c->max_tokens, c->max_batch);
  if (!(c->rms_eps > 0.f)) return fail(ANN_E_ARG, "rms_eps must be positive");
  if (!(c->attn_scale > 0.f) || c->attn_scale * Dh > 40.f)
    return fail(ANN_E_ARG, "attn_scale * head_dim must lie in (0, 40] (bounded-score softmax)");
  return ANN_OK;
}

}  // namespace

struct ann_ctx {
  ann_config c;
  int Dh;
  WLayout wl;
  SLayout sl;
  uint8_t* w = nullptr;
  uint8_t* kv = nullptr;
  uint8_t* ws = nullptr;
  bool bound = false;
  int len = 0;  // tokens held per sequence
  int B = 0;    // sequences held
  // decode-step graph (captured once per key, replayed every step)
  int graph_mode = -1;   // ANN_DECODE_GRAPH: 0 never, 1 always, unset: below GRAPH_MAX_B rows
  hipStream_t cap_st = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t gexec = nullptr;
  struct GKey {
    int B;
    const int32_t* tok;
    int32_t* out;
    float* logits;
    bool greedy;
    bool cand;
  } gkey{};
  bool cand_env = true;  // ANN_TOPK_CAND=0: the lm_head always stores z for the sampler
  // ANN_TOPK_VERIFY=1: the candidate sampler recomputes every lm_head tile and
  // flags (ann_check_device) any difference from the GEMM's candidates
  bool cand_verify = false;
  // host mirror of the device sampling parameters
  bool sp_valid = false;
  float sp_temp = 0.f;
  int sp_topk = 0;
  int sp_rows = 0;  // rows whose draw counters the last write set
  uint64_t sp_seed = 0, sp_step = 0;
  // persistent batch-1 decode step
  // work-groups of the persistent step (one per CU, on 3/4 of the CUs where
  // the model's rows fit that grid, else on all; 0: not possible; set on first use)
  int pd_g = -1;
  bool pd_env = true;    // ANN_PERSIST=0 disables
  bool pd_coop = false;  // ANN_PERSIST_COOP=1: cooperative launch
  // the persistent step's exchange area, the error word and the decode
  // attention's ticket counters and partials must be cleared before their
  // next user (a decode step or a one-token forward; clear_decode_state)
  bool dec_clear = true;
  // decode (batch >= 16): prefetch work-groups per attention launch that read
  // the next projections' weights ahead; -1 = not read yet, -2 = sized by
  // bytes, >= 0 = fixed by ANN_PREFETCH_WG
  int pf_wgs = -1;
  bool qa_env = true;      // ANN_QKV_ATTN: the fused qkv projection + decode attention
  uint32_t qa_tag = 0;     // tag of its last launch (0: none since the decode state was cleared)
  // decode attention: splits per (row, head) fixed by ANN_DEC_SPLITS (0: sized
  // by the batch, about 384 work-groups)
  int dec_split_env = 0;
  // rows the persistent step takes by default (0: by shape): its GEMV-style
  // phases apply every weight to each row in turn, so a row costs 40-60 us
  // more.  155M decode step at 1 / 2 / 3 / 4 rows, generic kernel: 185 / 256
  // / 308 / 370 us, against 258 / 301 / 320 / 326 us on the per-kernel path;
  // with the 155M instances 4 rows take 314 against 325 us (sampled 323
  // against 331), so that shape takes up to 4 rows, any other up to 3.
  // ANN_PERSIST_MAX_B (1..PD_MAX_B) fixes it
  int pd_max_b = 0;
  int pd_rep = PD_MAX_REP;   // copies of the persistent step's x' / x exchange
  int pd_on = 0;             // work-groups for the o rows (0: d / 8, 8 rows each)
  // one row: each head's qkv rows and attention splits on one XCD where the
  // shapes allow (ANN_PD_XCD=0: contiguous over the work-groups)
  bool pd_xcd_env = true;
  // the persistent step's compile-time instance for the 155M shape
  // (ANN_PD_SPECIALIZE=0: the generic kernel)
  bool pd_spec_env = true;
  // measurement: HIP event pairs around every launch of one kernel class
  int prof_kind = -1;
  std::vector<hipEvent_t> prof_ev;
  size_t prof_used = 0;

  const bf16_t* wptr(size_t off) const { return (const bf16_t*)(w + off); }
  const bf16_t* layer_w(int l, size_t off) const {
    return (const bf16_t*)(w + wl.layer0 + wl.layer_stride * l + off);
  }
  bf16_t* kcache(int l) const { return (bf16_t*)(kv + kv_layer_bytes(c) * l); }
  bf16_t* vcache(int l) const { return (bf16_t*)(kv + kv_layer_bytes(c) * (c.L + l)); }
  template <typename T> T* sp(size_t off) const { return (T*)(ws + off); }
  bool is_long(int l) const {
    for (int i = 0; i < c.n_long; ++i)
      if (c.long_layers[i] == l) return true;
    return false;
  }
};

namespace {

struct ProfScope {  // records an event pair around a launch of the profiled kind
  ann_ctx* c;
  hipStream_t st;
  bool on;
  ProfScope(ann_ctx* c_, int kind, hipStream_t st_) : c(c_), st(st_) {
    on = c->prof_kind == kind && c->prof_used + 2 <= c->prof_ev.size();
    if (on) hipEventRecord(c->prof_ev[c->prof_used], st);
  }
  ~ProfScope() {
    if (on) {
      hipEventRecord(c->prof_ev[c->prof_used + 1], st);
      c->prof_used += 2;
    }
  }
};

// y = pre(X) @ W^T for M rows with the given epilogue.
// Whether proj() routes an (M, N, K) projection to the large-tile MFMA GEMM.
bool proj_is_gemm(int M, int N, int K, int pre) {
  // the skinny GEMM re-reads W per 16 rows and A per 16 columns: wide
  // outputs (lm_head) go to the large-tile GEMM
  return !gemv_routes(M, K) && !(N <= 8 * K && gemm_skinny_fits(M, N, K, pre == PRE_RMS));
}

int proj(ann_ctx* c, int kind, int epi, int pre, const bf16_t* W, const bf16_t* X, int ldx,
         int M, int N, int K, EpiArgs ea, hipStream_t st) {
  // the QKV and CE epilogues exist on the MFMA GEMM only
  const bool gemm_only = epi == EPI_CE || epi == EPI_TOPK;
  const bool use_gemv = !gemm_only && gemv_routes(M, K);
  const bool use_sk = !gemm_only && !use_gemv && !proj_is_gemm(M, N, K, pre);
  if (epi == EPI_QKV && (use_gemv || use_sk)) return fail(ANN_E_ARG, "fused QKV needs the MFMA GEMM");
  // 65-128 rows with an RMS prologue and a plain-store epilogue (qkv, fc):
  // rms_apply + 64 x 64 MFMA tiles beat the skinny kernel's in-kernel RMS
  // (cfg5 decode 3.99 -> 3.88 ms per step, measured); up to 64 rows the
  // skinny kernel stays ahead
  const bool use_d64 = use_sk && pre == PRE_RMS && M > 64 && (epi == EPI_STORE || epi == EPI_RELU2);
  if (pre == PRE_RMS && !use_gemv && (!use_sk || use_d64)) {   // A normalised once into h
    if (K > c->c.d) return fail(ANN_E_ARG, "RMS prologue wider than the model dim");
    bf16_t* h = c->sp<bf16_t>(c->sl.hn);
    HIPCHK(rms_apply(X, ldx, h, K, M, K, c->c.rms_eps, st));
    X = h;
    ldx = K;
  }
  ProfScope ps(c, kind, st);
  if (use_gemv)
    HIPCHK(gemv(epi, pre, W, X, ldx, M, N, K, c->c.rms_eps, ea, st));
  else if (use_d64)
    HIPCHK(gemm_decode64(epi, X, ldx, W, M, N, K, ea, st));
  else if (use_sk)
    HIPCHK(gemm_skinny(epi, pre == PRE_RMS, X, ldx, W, M, N, K, c->c.rms_eps, ea, st));
  else
    HIPCHK(gemm(epi, X, ldx, W, M, N, K, ea, st));
  return ANN_OK;
}

// Split count of the decode attention: about 384 work-groups (1.5 per CU:
// more splits cost a partial round trip each and measured slower at batch
// 64), at most one 64-key chunk per split of the longest key range.
// Independent of the current length, so a captured step replays at every
// position.
int dec_splits(const ann_ctx* c, bool lng, int B) {
  const ann_config& g = c->c;
  const int keys = lng ? g.max_ctx : (g.window < g.max_ctx ? g.window : g.max_ctx);
  int n = (keys + 63) / 64;
  if (n > MAX_SPLIT) n = MAX_SPLIT;
  const int want = c->dec_split_env > 0 ? c->dec_split_env : (384 + B * g.H - 1) / (B * g.H);
  if (n > want) n = want;
  return n < 1 ? 1 : n;
}

// Prefetch work-groups per decode attention launch at batch B reading
// `bytes`: only where the attention itself is long enough to hide the extra
// reads (B >= 16), one work-group per 128 KB, 32..512.  Measured per step:
// 155M B=64 596 -> 575 us (flat over 48..192 work-groups), B=16 at ctx 8192
// 540 -> 522 us, 834M B=128 3766 -> 3550 us (48 work-groups: 3995 us, the
// reads outlast the attention).  ANN_PREFETCH_WG=n fixes the count (0: off).
int prefetch_wgs(ann_ctx* c, int B, size_t bytes) {
  if (c->pf_wgs == -1) {
    const char* e = getenv("ANN_PREFETCH_WG");
    c->pf_wgs = e ? atoi(e) : -2;
    if (e && c->pf_wgs < 0) c->pf_wgs = 0;
    if (c->pf_wgs > 1024) c->pf_wgs = 1024;
  }
  if (B < 16) return 0;
  if (c->pf_wgs >= 0) return c->pf_wgs;
  const size_t n = bytes >> 17;
  return n < 32 ? 32 : n > 512 ? 512 : (int)n;
}

// Zero the decode state once after ann_bind, before the first launch that
// uses it: the persistent step's exchange area (tags, generation, error word),
// the decode attention's ticket counters and its split partials.  That first
// launch is a decode step, or a forward of one token per sequence (its
// attention is the decode kernel too).  Never inside a graph capture: a
// captured decode step only follows a decode step that has cleared.
int clear_decode_state(ann_ctx* c, hipStream_t st) {
  if (!c->dec_clear) return ANN_OK;
  const ann_config& g = c->c;
  HIPCHK(hipMemsetAsync(c->ws + c->sl.pd, 0, c->sl.pd_bytes, st));
  HIPCHK(hipMemsetAsync(c->ws + c->sl.acnt, 0, (size_t)g.max_batch * g.H * 4, st));
  HIPCHK(hipMemsetAsync(c->ws + c->sl.part, 0,
                        (size_t)g.max_batch * g.H * MAX_SPLIT * (c->Dh + 1) * 8, st));
  HIPCHK(hipMemsetAsync(c->ws + c->sl.qat, 0, (size_t)g.max_batch * 3 * g.d / 2 * 8, st));
  c->qa_tag = 0;
  c->dec_clear = false;
  return ANN_OK;
}

// embed + all layers for M = B*T rows whose positions start at pos[b].
constexpr int GRAPH_MAX_B = 16;

int run_body(ann_ctx* c, const int32_t* tokens, int B, int T, hipStream_t st) {
  const ann_config& g = c->c;
  const int M = B * T, d = g.d, H = g.H, Dh = c->Dh;
  if (T == 1) {   // the decode attention's counters and partials start from zero
    const int rc0 = clear_decode_state(c, st);
    if (rc0) return rc0;
  }
  bf16_t* x = c->sp<bf16_t>(c->sl.x);
  bf16_t* x0 = c->sp<bf16_t>(c->sl.x0);
  bf16_t* qkv = c->sp<bf16_t>(c->sl.qkv);
  bf16_t* q = c->sp<bf16_t>(c->sl.q);
  bf16_t* ao = c->sp<bf16_t>(c->sl.ao);
  bf16_t* hid = c->sp<bf16_t>(c->sl.hid);
  u64* part = c->sp<u64>(c->sl.part);
  unsigned* err = (unsigned*)(c->ws + c->sl.pd + pd_layout(g, 8));
  const int32_t* pos = c->sp<int32_t>(c->sl.pos);
  const float* lam = (const float*)(c->w + c->wl.lam);
  const float* cs = (const float*)(c->w + c->wl.cs);
  const float* sn = (const float*)(c->w + c->wl.sn);

  HIPCHK(embed_rms(tokens, c->wptr(c->wl.embed), x, x0, M, d, g.V, g.rms_eps, st));
  for (int l = 0; l < g.L; ++l) {
    const bool lng = c->is_long(l);
    EpiArgs ea{};
    ea.out = qkv;
    ea.ldo = 3 * d;
    // prefill on the MFMA GEMM: QK-norm, RoPE and the cache append run in the
    // projection's epilogue (q lands in its own buffer, qkv is not written)
    ea.kc = c->kcache(l);
    ea.vc = c->vcache(l);
    ea.pos = pos;
    ea.cs = cs;
    ea.sn = sn;
    ea.T = T;
    ea.H = H;
    ea.Dh = Dh;
    ea.max_ctx = g.max_ctx;
    ea.eps = g.rms_eps;
    bool fuse_qkv = false;
    if (T > 1 && proj_is_gemm(M, 3 * d, d, PRE_RMS)) {
      EpiArgs fq = ea;
      fq.out = q;
      fq.ldo = d;
      if (gemm_qkv_fits(M, 3 * d, d, fq)) {
        ea = fq;
        fuse_qkv = true;
      }
    }
    // decode of 16..64 rows launched directly: the qkv projection and the
    // attention as one launch (qkv_attn_decode); never inside a graph
    // capture (its tag comes from a host counter) or a per-kernel profile
    bool fuse_qa = T == 1 && c->qa_env && c->prof_kind < 0 && qkv_attn_fits(B, d, Dh);
    if (fuse_qa) {
      hipStreamCaptureStatus cst = hipStreamCaptureStatusNone;
      HIPCHK(hipStreamIsCapturing(st, &cst));
      fuse_qa = cst == hipStreamCaptureStatusNone;
    }
    int rc = ANN_OK;
    if (!fuse_qa) {
      rc = proj(c, ANN_PROF_QKV, fuse_qkv ? EPI_QKV : EPI_STORE, PRE_RMS,
                c->layer_w(l, c->wl.qkv), x, d, M, 3 * d, d, ea, st);
      if (rc) return rc;
    }
    EpiArgs er{};
    er.x = x;
    er.x0 = x0;
    er.ldr = d;
    er.lam = lam + 8 * l;
    if (T == 1) {  // decode: fused QK-norm / RoPE / KV append and split combine
      const int ns = dec_splits(c, lng, B);
      // while the attention streams the KV cache, extra work-groups read this
      // layer's o / fc / proj weights and the next layer's qkv (contiguous
      // from o) so the projections find them in the memory-side cache
      WeightPrefetch pf;
      const size_t pfb = c->wl.layer_stride - (l + 1 < g.L ? 0 : c->wl.o);
      const int pfw = prefetch_wgs(c, B, pfb);
      if (pfw > 0) {
        pf.p = c->layer_w(l, c->wl.o);
        pf.bytes = pfb;
        pf.slices = (pfw + ns * H - 1) / (ns * H);
        pf.sink = c->sp<unsigned long long>(c->sl.pfsink);
      }
      if (fuse_qa) {
        c->qa_tag += 1;
        HIPCHK(qkv_attn_decode(x, c->layer_w(l, c->wl.qkv), c->sp<u64>(c->sl.qat), c->qa_tag,
                               c->kcache(l), c->vcache(l), pos, cs, sn, part,
                               c->sp<unsigned>(c->sl.acnt), err, ao, B, H, Dh, g.max_ctx,
                               g.window, lng, g.attn_scale, g.rms_eps, ns, pf, st));
      } else {
        ProfScope ps(c, ANN_PROF_ATTN, st);
        HIPCHK(attn_decode(qkv, c->kcache(l), c->vcache(l), pos, cs, sn, part,
                           c->sp<unsigned>(c->sl.acnt), err, ao, B, H, Dh, g.max_ctx, g.window, lng,
                           g.attn_scale, g.rms_eps, ns, pf, st));
      }
      rc = proj(c, ANN_PROF_O, EPI_RESID_ATTN, PRE_PLAIN, c->layer_w(l, c->wl.o), ao, d, M, d, d,
                er, st);
      if (rc) return rc;
    } else {
      if (!fuse_qkv)
        HIPCHK(qkv_post(qkv, q, c->kcache(l), c->vcache(l), pos, cs, sn, M, T, H, Dh, g.max_ctx,
                        g.rms_eps, st));
      {
        ProfScope ps(c, ANN_PROF_ATTN, st);
        HIPCHK(attn_prefill(q, c->kcache(l), c->vcache(l), pos, ao, B, T, H, Dh, g.max_ctx,
                            g.window, lng, g.attn_scale, st));
      }
      rc = proj(c, ANN_PROF_O, EPI_RESID_ATTN, PRE_PLAIN, c->layer_w(l, c->wl.o), ao, d, M, d, d,
                er, st);
      if (rc) return rc;
    }
    EpiArgs eh{};
    eh.out = hid;
    eh.ldo = 4 * d;
    rc = proj(c, ANN_PROF_FC, EPI_RELU2, PRE_RMS, c->layer_w(l, c->wl.fc), x, d, M, 4 * d, d, eh,
              st);
    if (rc) return rc;
    rc = proj(c, ANN_PROF_PROJ, EPI_RESID_MLP, PRE_PLAIN, c->layer_w(l, c->wl.proj), hid, 4 * d, M,
              d, 4 * d, er, st);
    if (rc) return rc;
  }
  return ANN_OK;
}

int check_ready(const ann_ctx* c) {
  if (!c) return fail(ANN_E_ARG, "context is null");
  if (!c->bound) return fail(ANN_E_STATE, "buffers not bound (call ann_bind first)");
  return ANN_OK;
}

int check_sampling(const ann_ctx* c, const ann_sampling* s) {
  if (!s) return fail(ANN_E_ARG, "sampling is null");
  if (!(s->temperature >= 0.f) || s->temperature != s->temperature)
    return fail(ANN_E_ARG, "temperature must be >= 0");
  // the samplers read z rows in 16-byte chunks
  if (s->temperature != 0.f && c->c.V % 8)
    return fail(ANN_E_ARG, "sampling (temperature > 0) needs V a multiple of 8 (V=%d)", c->c.V);
  return ANN_OK;
}

// The device error word: bounded waits that gave up (bit 0), the candidate
// sampler's check (bit 1).
unsigned* dec_err_word(ann_ctx* c) { return (unsigned*)(c->ws + c->sl.pd + pd_layout(c->c, 8)); }

// The lm_head stores top-k candidates (EPI_TOPK) and sample_cand draws from
// them -- no z -- where the MFMA GEMM takes the lm_head (3 .. 511 rows; up
// to 2 rows the GEMV keeps its own argmax keys) for greedy rows and for
// 1 <= top_k <= 256; top_k 0 (every entry kept) or larger samples from z.
bool cand_route(const ann_ctx* c, int B, bool greedy) {
  const ann_config& g = c->c;
  if (!c->cand_env || B >= 512 || !proj_is_gemm(B, g.V, g.d, PRE_RMS) || g.V > 65536) return false;
  return greedy || (c->sp_topk >= 1 && c->sp_topk <= 256 && c->sp_topk < g.V_sample);
}

// lm_head of the last row of each sequence -> sampled token (from the top-k
// candidates where cand_route says so, else from z); positions advance by
// pos_adv (the tokens this call added).  Sampling parameters come from the
// device copy written by sync_sampling.
int head_and_sample(ann_ctx* c, int B, int T, bool greedy, int32_t* out_tok, float* logits,
                    int pos_adv, hipStream_t st) {
  const ann_config& g = c->c;
  bf16_t* x = c->sp<bf16_t>(c->sl.x);
  bf16_t* zb = c->sp<bf16_t>(c->sl.zb);
  int32_t* pos = c->sp<int32_t>(c->sl.pos);
  EpiArgs ez{};
  ez.logits = logits;
  ez.ldz = g.V;
  if (cand_route(c, B, greedy)) {
    // candidates in the z area: (B, nt, TK_M) words, then (B, nt)
    const int nt = ce_tiles(g);
    uint32_t* cand = (uint32_t*)zb;
    uint32_t* cand_r = cand + (size_t)B * nt * TK_M;
    ez.cand = cand;
    ez.cand_r = cand_r;
    ez.nt = nt;
    ez.tk_first = greedy ? 1 : 0;
    ez.Vs = g.V_sample;
    int rc = proj(c, ANN_PROF_LM_HEAD, EPI_TOPK, PRE_RMS, c->wptr(c->wl.head),
                  x + (size_t)(T - 1) * g.d, T * g.d, B, g.V, g.d, ez, st);
    if (rc) return rc;
    // the GEMM's A operand: the rows normalised into hn by proj()
    HIPCHK(sample_cand(cand, cand_r, nt, (g.V_sample + 127) / 128, B, g.V_sample, nullptr,
                       c->sp<bf16_t>(c->sl.hn), g.d, c->wptr(c->wl.head), g.V, g.d,
                       c->sp<SampParams>(c->sl.sp),
                       c->sp<unsigned long long>(c->sl.steps), out_tok, pos, pos_adv,
                       c->cand_verify ? dec_err_word(c) : nullptr, st));
    return ANN_OK;
  }
  const bool fused_greedy = greedy && gemv_routes(B, g.d);
  unsigned long long* keys = c->sp<unsigned long long>(c->sl.amax);
  if (fused_greedy) {
    ez.amax = keys;
    ez.Vs = g.V_sample;
  } else {
    ez.z = zb;
  }
  int rc = proj(c, ANN_PROF_LM_HEAD, EPI_LOGITS, PRE_RMS, c->wptr(c->wl.head),
                x + (size_t)(T - 1) * g.d, T * g.d, B, g.V, g.d, ez, st);
  if (rc) return rc;
  if (fused_greedy)
    HIPCHK(argmax_finalize(keys, gemv_blocks(g.V, g.d), B, out_tok, pos, pos_adv, st));
  else
    HIPCHK(sample(zb, g.V, B, g.V_sample, c->sp<SampParams>(c->sl.sp),
                  c->sp<unsigned long long>(c->sl.steps), out_tok, pos, pos_adv, st));
  return ANN_OK;
}

// Bring the device sampling parameters / draw counters in line with s.  The
// sampler kernel reads the temperature from the device (0 = greedy, which it
// also serves above 8 rows), so a greedy call after a sampled one must write
// it; greedy draws nothing, so its seed / step / counters need not match.
// The counters cover the rows of the last write: a call with more rows writes.
int sync_sampling(ann_ctx* c, const ann_sampling* s, int B, hipStream_t st) {
  const bool greedy = s->temperature == 0.f;
  if (c->sp_valid && c->sp_temp == s->temperature &&
      (greedy || (c->sp_topk == s->top_k && c->sp_seed == s->seed && c->sp_step == s->step &&
                  B <= c->sp_rows)))
    return ANN_OK;
  HIPCHK(set_sampling(c->sp<SampParams>(c->sl.sp), c->sp<unsigned long long>(c->sl.steps), B,
                      s->temperature, s->top_k, s->seed, s->step, st));
  c->sp_valid = true;
  c->sp_temp = s->temperature;
  c->sp_topk = s->top_k;
  c->sp_seed = s->seed;
  c->sp_step = s->step;
  c->sp_rows = B;
  return ANN_OK;
}

void drop_graph(ann_ctx* c) {
  if (c->gexec) (void)hipGraphExecDestroy(c->gexec);
  if (c->graph) (void)hipGraphDestroy(c->graph);
  c->gexec = nullptr;
  c->graph = nullptr;
}

// Splits per (b, h) of the persistent step's attention: about 128 keys per
// work-group (one 16-key chunk per wave, issued before the wait for q/k/v).
// Above one row the B * H * s attention work-groups leave the o projection
// its d / 8 work-groups (ANN_PD_ON sets the count) and the split partials fit
// the LDS beside the row buffers.
int pd_splits(const ann_ctx* c, int B, bool lng) {
  const int keys = lng ? c->c.max_ctx : (c->c.window < c->c.max_ctx ? c->c.window : c->c.max_ctx);
  int s = (keys + 127) / 128;
  if (s > PD_MAX_SLONG) s = PD_MAX_SLONG;
  if (c->pd_g > 0 && s > c->pd_g / (B * c->c.H)) s = c->pd_g / (B * c->c.H);
  if (B > 1 && c->pd_g > 0) {
    const int on = c->pd_on > 0 ? c->pd_on : c->c.d / 8;
    const int cap = (c->pd_g - on) / (B * c->c.H);
    if (s > cap) s = cap;
    while (s > 1 && decode_persist_lds(B, c->c.d, c->c.H, c->Dh, s) > PD_MAX_LDS) --s;
  }
  return s < 1 ? 1 : s;
}

// Whether this decode step runs as the persistent kernel.
bool persist_ok(ann_ctx* c, int B) {
  const int max_b = c->pd_max_b > 0 ? c->pd_max_b
                    : (c->pd_spec_env && c->c.d == 768 && c->c.H == 6 && c->Dh == 128) ? 4 : 3;
  if (!c->pd_env || B < 1 || B > max_b ||
      (c->prof_kind >= 0 && c->prof_kind != ANN_PROF_STEP))
    return false;
  const ann_config& g = c->c;
  if (c->pd_g < 0) {
    int dev = 0, n = 0, coop = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess)
      n = 0;
    // Fewer work-groups than CUs exchange faster, and a count dividing d/2
    // (every projection's row pairs) keeps the work-groups equal: 155M
    // batch-1 step 216 us on 256 work-groups, 203.4 on 192, 207.9 on 184 and
    // 200, 208.7 on 176, 209.5 on 208, 209.1 on 128 (measured).  Default: the
    // largest divisor of d/2 up to 3/4 of the CUs; ANN_PERSIST_G=n sets it.
    int pick = 0;
    if (coop && n > 0 && n <= PD_MAX_G) {
      const char* ge = getenv("ANN_PERSIST_G");
      int want = 0;
      if (ge && atoi(ge) > 0) {
        want = atoi(ge) < n ? atoi(ge) : n;
      } else {
        for (int q = n * 3 / 4; q >= 1 && !want; --q)
          if ((g.d / 2) % q == 0) want = q;
      }
      const int cands[2] = {want, n};
      for (int cand : cands) {
        if (cand < 1) continue;
        c->pd_g = cand;   // pd_splits reads it
        if (decode_persist_fits(1, g.d, g.H, c->Dh, g.V, g.L, cand, pd_splits(c, 1, true))) {
          pick = cand;
          break;
        }
      }
    }
    c->pd_g = pick;
  }
  return c->pd_g > 0 && g.n_long <= 8 &&
         decode_persist_fits(B, g.d, g.H, c->Dh, g.V, g.L, c->pd_g, pd_splits(c, B, true));
}

int enqueue_persist(ann_ctx* c, const int32_t* tokens, int B, bool greedy, int32_t* out_tok,
                    float* logits, hipStream_t st) {
  const ann_config& g = c->c;
  PDParams P{};
  P.emb = c->wptr(c->wl.embed);
  P.head = c->wptr(c->wl.head);
  P.layers = c->layer_w(0, 0);
  P.lstride = c->wl.layer_stride / 2;
  P.o_qkv = c->wl.qkv / 2;
  P.o_o = c->wl.o / 2;
  P.o_fc = c->wl.fc / 2;
  P.o_proj = c->wl.proj / 2;
  P.lam = (const float*)(c->w + c->wl.lam);
  P.cs = (const float*)(c->w + c->wl.cs);
  P.sn = (const float*)(c->w + c->wl.sn);
  P.kc = c->kcache(0);
  P.vc = c->vcache(0);
  P.kvl = kv_layer_bytes(g) / 2;
  P.long_mask = 0;
  for (int i = 0; i < g.n_long; ++i) P.long_mask |= 1ull << g.long_layers[i];
  P.tok = tokens;
  P.out_tok = out_tok;
  P.pos = c->sp<int32_t>(c->sl.pos);
  P.z = c->sp<bf16_t>(c->sl.zb);
  // sampled: the step also leaves each work-group's top-k candidates, the
  // sampler reads z only when they cannot prove the kept set
  const int G = c->pd_g, zrows = (g.V + G - 1) / G;
  const bool cands = !greedy && c->cand_env && zrows <= 64 * PD_ZE && zrows <= 4 * g.d;
  if (cands) {
    P.cand = c->sp<uint32_t>(c->sl.pcand);
    P.cand_r = P.cand + (size_t)PD_MAX_B * PD_MAX_G * TK_M;
  }
  P.logits = logits;
  uint8_t* pd = c->ws + c->sl.pd;
  P.xq = (u64*)(pd + pd_layout(g, 1));
  P.xp = (u64*)(pd + pd_layout(g, 2));
  P.xm = (u64*)(pd + pd_layout(g, 3));
  P.xh = (u64*)(pd + pd_layout(g, 4));
  P.xx = (u64*)(pd + pd_layout(g, 5));
  P.xk = (u64*)(pd + pd_layout(g, 6));
  P.gen = (unsigned*)(pd + pd_layout(g, 7));
  P.err = (unsigned*)(pd + pd_layout(g, 8));
  P.d = g.d;
  P.H = g.H;
  P.L = g.L;
  P.V = g.V;
  P.Vs = g.V_sample;
  P.max_ctx = g.max_ctx;
  P.window = g.window;
  P.s_win = pd_splits(c, B, false);
  P.s_long = pd_splits(c, B, true);
  P.greedy = greedy ? 1 : 0;
  P.rep = c->pd_rep;
  P.on = c->pd_on > 0 ? c->pd_on : g.d / 8;
  P.rep_stride = (int)pd_rep_stride(g.d);
  P.h_stride = (int)pd_h_stride(g.d);
  P.p_stride = (int)pd_p_stride(g.d, g.H);
  P.head_xcd = c->pd_xcd_env && decode_persist_xcd_ok(B, g.d, g.H, c->Dh, G, P.s_long) ? 1 : 0;
  P.scale = g.attn_scale;
  P.shift = g.attn_scale * (float)c->Dh * 1.02f;
  P.eps = g.rms_eps;
  {
    ProfScope ps(c, ANN_PROF_STEP, st);
    HIPCHK(decode_persist(P, B, c->Dh, c->pd_g, c->pd_coop, c->pd_spec_env, st));
  }
  if (cands) {
    int holders = 0;   // work-groups whose rows start below Vs
    while (holders < G && (long long)g.V * holders / G < g.V_sample) ++holders;
    // the tiles' records are (row, work-group): row stride G
    HIPCHK(sample_cand(P.cand, P.cand_r, G, holders, B, g.V_sample, P.z, nullptr, 0, nullptr,
                       g.V, g.d, c->sp<SampParams>(c->sl.sp),
                       c->sp<unsigned long long>(c->sl.steps), out_tok, c->sp<int32_t>(c->sl.pos),
                       1, nullptr, st));
  } else if (!greedy) {
    HIPCHK(sample(c->sp<bf16_t>(c->sl.zb), g.V, B, g.V_sample, c->sp<SampParams>(c->sl.sp),
                  c->sp<unsigned long long>(c->sl.steps), out_tok, c->sp<int32_t>(c->sl.pos), 1,
                  st));
  }
  return ANN_OK;
}

int enqueue_decode(ann_ctx* c, const int32_t* tokens, int B, bool greedy, int32_t* out_tok,
                   float* logits, hipStream_t st) {
  if (persist_ok(c, B)) return enqueue_persist(c, tokens, B, greedy, out_tok, logits, st);
  int rc = run_body(c, tokens, B, 1, st);
  if (rc) return rc;
  return head_and_sample(c, B, 1, greedy, out_tok, logits, 1, st);
}

// Capture one decode step into a graph (once per key) and launch it.
int decode_graph(ann_ctx* c, const int32_t* tokens, int B, bool greedy, int32_t* out_tok,
                 float* logits, hipStream_t st) {
  const ann_ctx::GKey key{B, tokens, out_tok, logits, greedy, cand_route(c, B, greedy)};
  const bool same = c->gexec && key.B == c->gkey.B && key.tok == c->gkey.tok &&
                    key.out == c->gkey.out && key.logits == c->gkey.logits &&
                    key.greedy == c->gkey.greedy && key.cand == c->gkey.cand;
  if (!same) {
    drop_graph(c);
    if (!c->cap_st) HIPCHK(hipStreamCreateWithFlags(&c->cap_st, hipStreamNonBlocking));
    HIPCHK(hipStreamBeginCapture(c->cap_st, hipStreamCaptureModeThreadLocal));
    int rc = enqueue_decode(c, tokens, B, greedy, out_tok, logits, c->cap_st);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(c->cap_st, &g);
    if (rc || e != hipSuccess) {
      if (g) (void)hipGraphDestroy(g);
      return rc ? rc : fail(ANN_E_HIP, "graph capture failed: %s", hipGetErrorString(e));
    }
    c->graph = g;
    HIPCHK(hipGraphInstantiate(&c->gexec, g, nullptr, nullptr, 0));
    c->gkey = key;
  }
  HIPCHK(hipGraphLaunch(c->gexec, st));
  return ANN_OK;
}

}  // namespace

extern "C" {

const char* ann_last_error(void) { return g_err.c_str(); }
int ann_version(void) { return 1; }

int ann_create(const ann_config* cfg, ann_ctx** out) {
  if (!out) return fail(ANN_E_ARG, "out is null");
  *out = nullptr;
  int rc = check_config(cfg);
  if (rc) return rc;
  ann_ctx* c = new ann_ctx();
  c->c = *cfg;
  c->Dh = cfg->d / cfg->H;
  c->wl = weight_layout(*cfg);
  c->sl = ws_layout(*cfg);
  const char* ge = getenv("ANN_DECODE_GRAPH");
  c->graph_mode = ge ? (ge[0] == '0' ? 0 : 1) : -1;
  const char* pe = getenv("ANN_PERSIST");
  c->pd_env = !(pe && pe[0] == '0');
  const char* on = getenv("ANN_PD_ON");
  c->pd_on = on && atoi(on) > 0 ? atoi(on) : 0;
  const char* px = getenv("ANN_PD_XCD");
  c->pd_xcd_env = !(px && px[0] == '0');
  const char* ps = getenv("ANN_PD_SPECIALIZE");
  c->pd_spec_env = !(ps && ps[0] == '0');
  const char* pr = getenv("ANN_PD_REP");
  if (pr && atoi(pr) >= 1 && atoi(pr) <= PD_MAX_REP) c->pd_rep = atoi(pr);
  const char* ds = getenv("ANN_DEC_SPLITS");
  c->dec_split_env = ds ? atoi(ds) : 0;
  if (c->dec_split_env < 0 || c->dec_split_env > MAX_SPLIT) c->dec_split_env = 0;
  const char* pm = getenv("ANN_PERSIST_MAX_B");
  if (pm && atoi(pm) >= 1 && atoi(pm) <= PD_MAX_B) c->pd_max_b = atoi(pm);
  const char* tc = getenv("ANN_TOPK_CAND");
  c->cand_env = !(tc && tc[0] == '0');
  const char* tv = getenv("ANN_TOPK_VERIFY");
  c->cand_verify = tv && tv[0] == '1';
  const char* qa = getenv("ANN_QKV_ATTN");
  c->qa_env = !(qa && qa[0] == '0');
  const char* pc = getenv("ANN_PERSIST_COOP");
  c->pd_coop = pc && pc[0] == '1';
  *out = c;
  return ANN_OK;
}

void ann_destroy(ann_ctx* ctx) {
  if (!ctx) return;
  for (hipEvent_t e : ctx->prof_ev) (void)hipEventDestroy(e);
  drop_graph(ctx);
  if (ctx->cap_st) (void)hipStreamDestroy(ctx->cap_st);
  delete ctx;
}

int ann_profile_enable(ann_ctx* c, int32_t kind, int32_t max_launches) {
  if (!c) return fail(ANN_E_ARG, "context is null");
  if (kind < -1 || kind > ANN_PROF_STEP) return fail(ANN_E_ARG, "bad kernel kind %d", kind);
  for (hipEvent_t e : c->prof_ev) (void)hipEventDestroy(e);
  c->prof_ev.clear();
  c->prof_used = 0;
  c->prof_kind = -1;
  if (kind < 0) return ANN_OK;
  if (max_launches <= 0) return fail(ANN_E_ARG, "max_launches must be positive");
  c->prof_ev.resize((size_t)max_launches * 2);
  for (auto& e : c->prof_ev) HIPCHK(hipEventCreate(&e));
  c->prof_kind = kind;
  return ANN_OK;
}

int ann_profile_read(ann_ctx* c, float* total_ms, int32_t* launches) {
  if (!c || !total_ms || !launches) return fail(ANN_E_ARG, "null argument");
  double tot = 0.0;
  for (size_t i = 0; i + 1 < c->prof_used; i += 2) {
    HIPCHK(hipEventSynchronize(c->prof_ev[i + 1]));
    float ms = 0.f;
    HIPCHK(hipEventElapsedTime(&ms, c->prof_ev[i], c->prof_ev[i + 1]));
    tot += ms;
  }
  *total_ms = (float)tot;
  *launches = (int32_t)(c->prof_used / 2);
  c->prof_used = 0;
  return ANN_OK;
}

int ann_check_device(ann_ctx* c, void* stream) {
  int rc = check_ready(c);
  if (rc) return rc;
  HIPCHK(hipStreamSynchronize((hipStream_t)stream));
  if (c->dec_clear) return ANN_OK;   // no decode-state user has run since binding
  unsigned* err = dec_err_word(c);
  unsigned h = 0;
  HIPCHK(hipMemcpy(&h, err, sizeof h, hipMemcpyDeviceToHost));
  if (h) {
    HIPCHK(hipMemset(err, 0, sizeof h));
    if (h & 2u)
      return fail(ANN_E_HIP, "sampler check: recomputed lm_head keys differ from the candidates");
    return fail(ANN_E_HIP, "decode step: a bounded cross-work-group wait timed out");
  }
  return ANN_OK;
}

size_t ann_weight_bytes(const ann_config* cfg) {
  return check_config(cfg) ? 0 : weight_layout(*cfg).total;
}

size_t ann_kv_bytes(const ann_config* cfg) {
  return check_config(cfg) ? 0 : kv_layer_bytes(*cfg) * 2 * cfg->L;
}

size_t ann_workspace_bytes(const ann_config* cfg) {
  return check_config(cfg) ? 0 : ws_layout(*cfg).total;
}

int ann_pack_weights(ann_ctx* c, const ann_params_f32* p, void* wbuf, size_t wbytes,
                     void* stream) {
  if (!c || !p || !wbuf) return fail(ANN_E_ARG, "null argument");
  if (wbytes < c->wl.total)
    return fail(ANN_E_CAPACITY, "weight buffer %zu bytes < required %zu", wbytes, c->wl.total);
  if (!p->embed || !p->lm_head || !p->attn_bank || !p->fc_bank || !p->proj_bank ||
      !p->resid_lambdas || !p->post_lambdas || !p->x0_lambdas || !p->sa_lambdas)
    return fail(ANN_E_ARG, "a parameter pointer is null");
  hipStream_t st = (hipStream_t)stream;
  const ann_config& g = c->c;
  const int d = g.d, V = g.V, L = g.L;
  uint8_t* w = (uint8_t*)wbuf;
  HIPCHK(pack_cast(p->embed, (bf16_t*)(w + c->wl.embed), (size_t)V * d, st));
  HIPCHK(pack_transpose(p->lm_head, (bf16_t*)(w + c->wl.head), d, V, d, nullptr, st));
  for (int l = 0; l < L; ++l) {
    uint8_t* lw = w + c->wl.layer0 + c->wl.layer_stride * l;
    const float* ab = p->attn_bank + (size_t)l * 4 * d * d;
    for (int j = 0; j < 3; ++j)
      HIPCHK(pack_transpose(ab + (size_t)j * d * d, (bf16_t*)(lw + c->wl.qkv) + (size_t)j * d * d,
                            d, d, d, p->sa_lambdas + 2 * l, st));
    HIPCHK(pack_transpose(ab + (size_t)3 * d * d, (bf16_t*)(lw + c->wl.o), d, d, d,
                          p->sa_lambdas + 2 * l + 1, st));
    HIPCHK(pack_transpose(p->fc_bank + (size_t)l * d * 4 * d, (bf16_t*)(lw + c->wl.fc), d, 4 * d,
                          d, nullptr, st));
    HIPCHK(pack_transpose(p->proj_bank + (size_t)l * 4 * d * d, (bf16_t*)(lw + c->wl.proj), 4 * d,
                          d, 4 * d, nullptr, st));
  }
  HIPCHK(pack_lambdas(p->resid_lambdas, p->post_lambdas, p->x0_lambdas, (float*)(w + c->wl.lam),
                      L, st));
  HIPCHK(rope_tables((float*)(w + c->wl.cs), (float*)(w + c->wl.sn), g.max_ctx, c->Dh,
                     g.rope_base, st));
  return ANN_OK;
}

int ann_bind(ann_ctx* c, void* wbuf, size_t wbytes, void* kv, size_t kvbytes, void* workspace,
             size_t wsbytes) {
  if (!c || !wbuf || !kv || !workspace) return fail(ANN_E_ARG, "null argument");
  if (wbytes < c->wl.total)
    return fail(ANN_E_CAPACITY, "weight buffer %zu bytes < required %zu", wbytes, c->wl.total);
  const size_t kvneed = kv_layer_bytes(c->c) * 2 * c->c.L;
  if (kvbytes < kvneed)
    return fail(ANN_E_CAPACITY, "kv buffer %zu bytes < required %zu", kvbytes, kvneed);
  if (wsbytes < c->sl.total)
    return fail(ANN_E_CAPACITY, "workspace %zu bytes < required %zu", wsbytes, c->sl.total);
  if (((uintptr_t)wbuf | (uintptr_t)kv | (uintptr_t)workspace) & 255)
    return fail(ANN_E_ARG, "buffers must be 256-byte aligned");
  drop_graph(c);
  c->sp_valid = false;
  c->w = (uint8_t*)wbuf;
  c->kv = (uint8_t*)kv;
  c->ws = (uint8_t*)workspace;
  c->dec_clear = true;
  c->bound = true;
  c->len = 0;
  c->B = 0;
  return ANN_OK;
}

int ann_reset(ann_ctx* c) {
  if (!c) return fail(ANN_E_ARG, "context is null");
  c->len = 0;
  c->B = 0;
  return ANN_OK;
}

int ann_context_length(const ann_ctx* c) { return c ? c->len : -1; }

static int check_prefill_shape(ann_ctx* c, const int32_t* tokens, int B, int T) {
  int rc = check_ready(c);
  if (rc) return rc;
  if (!tokens) return fail(ANN_E_ARG, "tokens is null");
  if (B < 1 || T < 1) return fail(ANN_E_ARG, "B=%d, T=%d must be >= 1", B, T);
  if (B > c->c.max_batch) return fail(ANN_E_CAPACITY, "B=%d > max_batch=%d", B, c->c.max_batch);
  if (T > c->c.max_ctx) return fail(ANN_E_CAPACITY, "T=%d > max_ctx=%d", T, c->c.max_ctx);
  if ((size_t)B * T > (size_t)c->c.max_tokens)
    return fail(ANN_E_CAPACITY, "B*T=%d > max_tokens=%d", B * T, c->c.max_tokens);
  return ANN_OK;
}

int ann_forward_logits(ann_ctx* c, const int32_t* tokens, int32_t B, int32_t T, float* logits,
                       void* stream) {
  int rc = check_prefill_shape(c, tokens, B, T);
  if (rc) return rc;
  if (!logits) return fail(ANN_E_ARG, "logits is null");
  hipStream_t st = (hipStream_t)stream;
  int32_t* pos = c->sp<int32_t>(c->sl.pos);
  HIPCHK(set_pos(pos, B, 0, st));
  c->len = 0;
  c->B = B;
  rc = run_body(c, tokens, B, T, st);
  if (rc) return rc;
  EpiArgs ez{};
  ez.logits = logits;
  ez.ldz = c->c.V;
  rc = proj(c, ANN_PROF_LM_HEAD, EPI_LOGITS, PRE_RMS, c->wptr(c->wl.head), c->sp<bf16_t>(c->sl.x),
            c->c.d, B * T, c->c.V, c->c.d, ez, st);
  if (rc) return rc;
  HIPCHK(advance_pos(pos, B, T, st));
  c->len = T;
  return ANN_OK;
}

int ann_forward_loss(ann_ctx* c, const int32_t* tokens, const int32_t* targets, int32_t B,
                     int32_t T, float* loss, float* row_loss, void* stream) {
  int rc = check_prefill_shape(c, tokens, B, T);
  if (rc) return rc;
  if (!targets || !loss) return fail(ANN_E_ARG, "targets / loss is null");
  hipStream_t st = (hipStream_t)stream;
  int32_t* pos = c->sp<int32_t>(c->sl.pos);
  HIPCHK(set_pos(pos, B, 0, st));
  c->len = 0;
  c->B = B;
  rc = run_body(c, tokens, B, T, st);
  if (rc) return rc;
  const int M = B * T;
  EpiArgs ec{};
  ec.ce_part = c->sp<float>(c->sl.ce);
  ec.ce_tz = c->sp<float>(c->sl.ce_tz);
  ec.tgt = targets;
  ec.ldz = M;
  rc = proj(c, ANN_PROF_LM_HEAD, EPI_CE, PRE_RMS, c->wptr(c->wl.head), c->sp<bf16_t>(c->sl.x),
            c->c.d, M, c->c.V, c->c.d, ec, st);
  if (rc) return rc;
  float* rows = row_loss ? row_loss : c->sp<float>(c->sl.ce_rows);
  HIPCHK(ce_finalize(ec.ce_part, M, ce_tiles(c->c), ec.ce_tz, M, rows, loss, st));
  HIPCHK(advance_pos(pos, B, T, st));
  c->len = T;
  return ANN_OK;
}

int ann_prefill(ann_ctx* c, const int32_t* tokens, int32_t B, int32_t T, const ann_sampling* s,
                int32_t* out_tok, float* logits, void* stream) {
  int rc = check_prefill_shape(c, tokens, B, T);
  if (rc) return rc;
  rc = check_sampling(c, s);
  if (rc) return rc;
  if (!out_tok) return fail(ANN_E_ARG, "out_tok is null");
  hipStream_t st = (hipStream_t)stream;
  int32_t* pos = c->sp<int32_t>(c->sl.pos);
  HIPCHK(set_pos(pos, B, 0, st));
  c->len = 0;
  c->B = B;
  rc = sync_sampling(c, s, B, st);
  if (rc) return rc;
  rc = run_body(c, tokens, B, T, st);
  if (rc) return rc;
  rc = head_and_sample(c, B, T, s->temperature == 0.f, out_tok, logits, T, st);
  if (rc) return rc;
  if (s->temperature != 0.f) c->sp_step += 1;
  c->len = T;
  return ANN_OK;
}

int ann_decode_step(ann_ctx* c, const int32_t* tokens, int32_t B, const ann_sampling* s,
                    int32_t* out_tok, float* logits, void* stream) {
  int rc = check_ready(c);
  if (rc) return rc;
  rc = check_sampling(c, s);
  if (rc) return rc;
  if (!tokens || !out_tok) return fail(ANN_E_ARG, "tokens / out_tok is null");
  if (c->len == 0) return fail(ANN_E_STATE, "no sequences: prefill first");
  if (B != c->B) return fail(ANN_E_ARG, "B=%d differs from the prefilled batch %d", B, c->B);
  if (c->len + 1 > c->c.max_ctx)
    return fail(ANN_E_CAPACITY, "context %d would exceed max_ctx=%d", c->len + 1, c->c.max_ctx);
  hipStream_t st = (hipStream_t)stream;
  rc = sync_sampling(c, s, B, st);
  if (rc) return rc;
  const bool greedy = s->temperature == 0.f;
  // set up before the step may be captured into a graph below
  if (cand_route(c, B, greedy)) HIPCHK(sample_prepare());
  rc = clear_decode_state(c, st);   // tags, tickets, partials and the error word
  if (rc) return rc;
  // The batch-1 persistent step is one kernel (plus the sampler when not
  // greedy): launched directly, measured 2.5% more tokens per second than
  // replaying it as a graph (0.2019 against 0.2070 ms per token at 155M).
  // The per-kernel path (tens of launches) replays its captured graph below
  // GRAPH_MAX_B rows; from there launched directly, ~4 us per step faster
  // (batch 64 557.4 -> 553.0 us, 16 x 8192 504.1 -> 500.1, 128 rows equal),
  // the host enqueueing a step well inside its GPU time.
  const bool graph = c->graph_mode == 1 || (c->graph_mode < 0 && B < GRAPH_MAX_B);
  if (graph && c->prof_kind < 0 && !persist_ok(c, B))
    rc = decode_graph(c, tokens, B, greedy, out_tok, logits, st);
  else
    rc = enqueue_decode(c, tokens, B, greedy, out_tok, logits, st);
  if (rc) return rc;
  if (!greedy) c->sp_step += 1;
  c->len += 1;
  return ANN_OK;
}

int ann_op_relu2(const void* x, void* y, size_t n, int32_t dtype, void* stream) {
  if ((!x || !y) && n) return fail(ANN_E_ARG, "null argument");
  if (dtype != ANN_DTYPE_F32 && dtype != ANN_DTYPE_BF16) return fail(ANN_E_ARG, "bad dtype");
  HIPCHK(op_relu2(x, y, n, dtype, (hipStream_t)stream));
  return ANN_OK;
}

int ann_op_rope_ht(const void* x, void* y, const float* cs, const float* sn, int32_t B, int32_t T,
                   int32_t H, int32_t D, int32_t pos0, int32_t inverse, int32_t dtype,
                   void* stream) {
  if (!x || !y || !cs || !sn) return fail(ANN_E_ARG, "null argument");
  if (B < 0 || T < 0 || H < 0 || D <= 0 || D % 4 || pos0 < 0)
    return fail(ANN_E_ARG, "bad shape B=%d T=%d H=%d D=%d pos0=%d", B, T, H, D, pos0);
  if (dtype != ANN_DTYPE_F32 && dtype != ANN_DTYPE_BF16) return fail(ANN_E_ARG, "bad dtype");
  HIPCHK(op_rope(x, y, cs, sn, B, T, H, D, pos0, inverse, dtype, (hipStream_t)stream));
  return ANN_OK;
}

int ann_op_rope_tables(float* cs, float* sn, int32_t seq_len, int32_t head_dim, float base,
                       void* stream) {
  if (!cs || !sn) return fail(ANN_E_ARG, "null argument");
  if (seq_len <= 0 || head_dim <= 0 || head_dim % 4 || !(base > 0.f))
    return fail(ANN_E_ARG, "bad table shape");
  HIPCHK(rope_tables(cs, sn, seq_len, head_dim, base, (hipStream_t)stream));
  return ANN_OK;
}

int ann_op_rms_norm(const void* x, void* y, int32_t rows, int32_t dim, float eps, int32_t dtype,
                    void* stream) {
  if (!x || !y) return fail(ANN_E_ARG, "null argument");
  if (rows < 0 || dim <= 0) return fail(ANN_E_ARG, "bad shape rows=%d dim=%d", rows, dim);
  if (dtype != ANN_DTYPE_F32 && dtype != ANN_DTYPE_BF16) return fail(ANN_E_ARG, "bad dtype");
  HIPCHK(op_rms(x, y, rows, dim, eps, dtype, (hipStream_t)stream));
  return ANN_OK;
}

// ---- optimizer step (muon.py, metal_kernels.py:236-328) -------------------------

int ann_op_adam_step(const float* p, const float* g, const float* m, const float* v, size_t n,
                     float beta1, float beta2, float eps, float step_size, float eff_wd,
                     float* p_out, float* m_out, float* v_out, void* stream) {
  if (n && (!p || !g || !m || !v || !p_out || !m_out || !v_out))
    return fail(ANN_E_ARG, "null argument");
  HIPCHK(adam_step(p, g, m, v, n, beta1, beta2, eps, step_size, eff_wd, p_out, m_out, v_out,
                   (hipStream_t)stream));
  return ANN_OK;
}

int ann_op_muon_momentum(const float* g, const float* buf, size_t n, float mu, float* geff,
                         float* buf_out, void* stream) {
  if (n && (!g || !buf || !geff || !buf_out)) return fail(ANN_E_ARG, "null argument");
  HIPCHK(muon_momentum(g, buf, n, mu, geff, buf_out, (hipStream_t)stream));
  return ANN_OK;
}

int ann_op_muon_apply(const float* p, const float* u, size_t n, float lr, float wd, float* p_out,
                      void* stream) {
  if (n && (!p || !u || !p_out)) return fail(ANN_E_ARG, "null argument");
  HIPCHK(muon_apply(p, u, n, lr, wd, p_out, (hipStream_t)stream));
  return ANN_OK;
}

size_t ann_op_polar_express_ws_bytes(int32_t batch, int32_t M, int32_t N) {
  return polar_express_ws_bytes(batch, M, N);
}

int ann_op_polar_express(const float* g, int32_t batch, int32_t M, int32_t N, void* out,
                         void* ws, size_t ws_bytes, void* stream) {
  if (!g || !out || !ws) return fail(ANN_E_ARG, "null argument");
  if (batch <= 0 || batch > 65535 || M <= 0 || N <= 0 || M % 64 || N % 64)
    return fail(ANN_E_ARG, "bad shape batch=%d M=%d N=%d (M, N multiples of 64)", batch, M, N);
  if (ws_bytes < polar_express_ws_bytes(batch, M, N))
    return fail(ANN_E_ARG, "workspace %zu < %zu bytes", ws_bytes,
                polar_express_ws_bytes(batch, M, N));
  HIPCHK(polar_express(g, batch, M, N, (bf16_t*)out, ws, ws_bytes, (hipStream_t)stream));
  return ANN_OK;
}

size_t ann_op_normuon_ws_bytes(int32_t batch, int32_t M, int32_t N) {
  return normuon_ws_bytes(batch, M, N);
}

int ann_op_normuon(const void* v, float* second_mom, int32_t batch, int32_t M, int32_t N,
                   float beta2, float* out, void* ws, size_t ws_bytes, void* stream) {
  if (!v || !second_mom || !out || !ws) return fail(ANN_E_ARG, "null argument");
  if (batch <= 0 || M <= 0 || N <= 0)
    return fail(ANN_E_ARG, "bad shape batch=%d M=%d N=%d", batch, M, N);
  if (ws_bytes < normuon_ws_bytes(batch, M, N))
    return fail(ANN_E_ARG, "workspace %zu < %zu bytes", ws_bytes, normuon_ws_bytes(batch, M, N));
  HIPCHK(normuon((const bf16_t*)v, second_mom, batch, M, N, beta2, out, ws, ws_bytes,
                 (hipStream_t)stream));
  return ANN_OK;
}

size_t ann_op_normuon_noalloc_max_bytes(void) { return NM_SCRATCH_BYTES; }

int ann_op_normuon_noalloc(const void* v, float* second_mom, int32_t batch, int32_t M, int32_t N,
                           float beta2, float* out, void* stream) {
  if (!v || !second_mom || !out) return fail(ANN_E_ARG, "null argument");
  if (batch <= 0 || M <= 0 || N <= 0)
    return fail(ANN_E_ARG, "bad shape batch=%d M=%d N=%d", batch, M, N);
  const size_t need = normuon_ws_bytes(batch, M, N);
  if (need > NM_SCRATCH_BYTES)
    return fail(ANN_E_CAPACITY,
                "normuon_noalloc: scratch of %zu bytes needed, the fixed array holds %zu "
                "(batch * max(M, N) up to %zu)",
                need, NM_SCRATCH_BYTES, NM_SCRATCH_BYTES / 8);
  const hipError_t e = normuon_noalloc((const bf16_t*)v, second_mom, batch, M, N, beta2, out,
                                       (hipStream_t)stream);
  if (e == hipErrorInvalidDevice)
    return fail(ANN_E_ARG, "normuon_noalloc: the stream must belong to the current device");
  if (e != hipSuccess) return fail(ANN_E_HIP, "normuon_noalloc: %s", hipGetErrorString(e));
  return ANN_OK;
}

}  // extern "C"
