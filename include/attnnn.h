/* attnnn.h -- C ABI of libattnnn.so, the gfx950 (MI355X) implementation of the
 * autoregressive token loop of attention_nn (sample.py running model.py).
 *
 * Plain C: pointers, sizes, ints.  No torch or C++ types cross this boundary.
 * Every entry point returns ANN_OK (0) or a negative ANN_E_* code; the message
 * of the last failure on the calling thread is ann_last_error().  Arguments
 * are validated on the host before any kernel is launched.
 *
 * Ownership: the caller allocates every device buffer (weights, KV cache,
 * workspace, inputs, outputs) and keeps it alive while a context uses it; the
 * library keeps raw pointers and never frees them.  A context owns host state
 * only.  One context per stream; calls on one context are not thread-safe.
 * Work is enqueued on the caller's hipStream_t (passed as void*); calls return
 * without synchronising unless noted.
 *
 * Reference interfaces replaced (henneberger/attention_nn):
 *   ann_create / ann_pack_weights / ann_bind  <- GPT(cfg) + params dict
 *                                                (model.py:138-153, sample.py:31-38)
 *   ann_forward_logits                        <- GPT.logits (model.py:223-263)
 *   ann_forward_loss                          <- GPT.__call__ (model.py:180-221) with the
 *                                                fused softcap CE (softcap_ce, model.py:
 *                                                121-132; ce_softcap_fwd, metal_kernels.py:
 *                                                153-193, 213-221)
 *   ann_prefill / ann_decode_step             <- the per-token loop body
 *                                                (sample.py:42-50: logits of the
 *                                                last row, /temp, top-k, categorical)
 *   ann_op_relu2                              <- relu2 (metal_kernels.py:37-47,62-68)
 *   ann_op_rope_ht                            <- rope_ht (metal_kernels.py:87-134)
 *   ann_op_rope_tables                        <- make_rope_tables (metal_kernels.py:144-150)
 *   ann_op_rms_norm                           <- rms (model.py:48-49)
 *   ann_op_adam_step                          <- adam_step (metal_kernels.py:241-270)
 *   ann_op_muon_momentum                      <- muon_momentum (metal_kernels.py:277-300)
 *   ann_op_muon_apply                         <- muon_apply (metal_kernels.py:306-329)
 *   ann_op_polar_express(_ws_bytes)           <- polar_express (muon.py:28-44)
 *   ann_op_normuon(_ws_bytes)                 <- normuon_rescale (muon.py:47-63)
 */
#ifndef ATTNNN_H
#define ATTNNN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ANN_OK 0
#define ANN_E_ARG (-1)      /* bad argument, shape or size */
#define ANN_E_STATE (-2)    /* call out of order (e.g. decode before prefill) */
#define ANN_E_CAPACITY (-3) /* batch / context / buffer exceeds what was bound */
#define ANN_E_HIP (-4)      /* a HIP runtime call failed */

#define ANN_MAX_LONG_LAYERS 8
#define ANN_DTYPE_F32 0
#define ANN_DTYPE_BF16 1

/* GPTConfig (model.py:30-45) plus the capacities the caller will bind. */
typedef struct ann_config {
  int32_t d;          /* model_dim */
  int32_t L;          /* num_layers */
  int32_t H;          /* num_heads; head_dim = d / H */
  int32_t V;          /* vocab_size (rows of embed / columns of lm_head) */
  int32_t V_sample;   /* rows sampling considers (50257, sample.py:45) */
  int32_t window;     /* sliding window of the short layers */
  int32_t n_long;     /* number of full-causal layers */
  int32_t long_layers[ANN_MAX_LONG_LAYERS];
  float attn_scale;   /* 0.1 */
  float rope_base;    /* 1024 */
  float rms_eps;      /* 1e-6 */
  int32_t max_batch;  /* sequences per call */
  int32_t max_ctx;    /* KV-cache length per sequence; also RoPE table length */
  int32_t max_tokens; /* rows per forward call (B*T of the largest prefill) */
} ann_config;

/* Device pointers to the reference fp32 parameter dict (model.py:52-77). */
typedef struct ann_params_f32 {
  const float* embed;         /* (V, d) */
  const float* lm_head;       /* (d, V) */
  const float* attn_bank;     /* (L, 4, d, d): q, k, v, o, each (in, out) */
  const float* fc_bank;       /* (L, d, 4d) */
  const float* proj_bank;     /* (L, 4d, d) */
  const float* resid_lambdas; /* (L, 2) */
  const float* post_lambdas;  /* (L, 2) */
  const float* x0_lambdas;    /* (L,) */
  const float* sa_lambdas;    /* (L, 2) */
} ann_params_f32;

/* Sampling of one step (sample.py:45-49).  temperature == 0 selects greedy
 * (argmax over the first V_sample logits, lowest index on ties).  top_k <= 0
 * or >= V_sample keeps every row.  Draws use Philox4x32-10 with counter
 * (step, row) and key seed. */
typedef struct ann_sampling {
  float temperature;
  int32_t top_k;
  uint64_t seed;
  uint64_t step;
} ann_sampling;

typedef struct ann_ctx ann_ctx;

const char* ann_last_error(void);
int ann_version(void);

/* Validate cfg and create a context (host state only). */
int ann_create(const ann_config* cfg, ann_ctx** out);
void ann_destroy(ann_ctx* ctx);

/* Bytes the caller must allocate for each device buffer. */
size_t ann_weight_bytes(const ann_config* cfg);
size_t ann_kv_bytes(const ann_config* cfg);
size_t ann_workspace_bytes(const ann_config* cfg);

/* Convert the fp32 parameter dict (device pointers) into the packed bf16
 * layout in wbuf (ann_weight_bytes bytes): bf16 casts, sa_lambdas folded into
 * the QKV / O weights with the two roundings of model.py:239-241, every
 * matrix stored (out, in) so a row of the output is a contiguous dot product,
 * RoPE tables appended.  Enqueued on stream. */
int ann_pack_weights(ann_ctx* ctx, const ann_params_f32* src, void* wbuf,
                     size_t wbytes, void* stream);

/* Attach the caller's buffers; sizes are checked against the ann_*_bytes. */
int ann_bind(ann_ctx* ctx, void* wbuf, size_t wbytes, void* kv, size_t kvbytes,
             void* workspace, size_t wsbytes);

/* Forget all sequences (the next call must be a prefill). */
int ann_reset(ann_ctx* ctx);

/* GPT.logits: tokens (B, T) int32 at positions 0..T-1 -> softcapped fp32
 * logits (B, T, V).  Leaves the KV cache filled for those B sequences, so
 * ann_decode_step may follow. */
int ann_forward_logits(ann_ctx* ctx, const int32_t* tokens, int32_t B, int32_t T,
                       float* logits, void* stream);

/* GPT.__call__ (training forward, loss only): tokens and targets (B, T) int32
 * on the device, positions 0..T-1.  Writes the mean over the B*T rows of
 * log(sum_v exp(zc[v])) - zc[target], zc = 23*sigmoid((z + 5)/7.5) and
 * z = bf16(rms(x) @ lm_head) over all V columns, as one fp32 to *loss, and the
 * per-row losses (B*T fp32) to row_loss when non-null.  The logits never
 * reach memory.  Targets must lie in [0, V) (not checked on the device: an
 * out-of-range target leaves its row's value undefined).  Leaves the KV cache
 * filled like ann_forward_logits. */
int ann_forward_loss(ann_ctx* ctx, const int32_t* tokens, const int32_t* targets, int32_t B,
                     int32_t T, float* loss, float* row_loss, void* stream);

/* Prefill B prompts of T tokens (positions 0..T-1), then sample one token
 * per sequence into out_tok (B).  logits (B, V) of the last rows is written
 * when non-null. */
int ann_prefill(ann_ctx* ctx, const int32_t* tokens, int32_t B, int32_t T,
                const ann_sampling* s, int32_t* out_tok, float* logits,
                void* stream);

/* One decode step: tokens (B) are appended at each sequence's next position,
 * one token per sequence is sampled into out_tok (B).  out_tok may equal
 * tokens.  logits (B, V) written when non-null. */
int ann_decode_step(ann_ctx* ctx, const int32_t* tokens, int32_t B,
                    const ann_sampling* s, int32_t* out_tok, float* logits,
                    void* stream);

/* Current length of the bound sequences (host mirror; 0 after reset). */
int ann_context_length(const ann_ctx* ctx);

/* ---- operators (the reference's kernel-level API) --------------------- */

/* y = max(x, 0)^2 computed in fp32, stored in dtype; n elements. */
int ann_op_relu2(const void* x, void* y, size_t n, int32_t dtype, void* stream);

/* Half-truncated RoPE of x (B, T, H, D) in dtype: pairs (2p, 2p+1), p < D/4,
 * rotated by the angle of position pos0 + t from the fp32 tables cs, sn
 * (rows >= pos0 + T, D/4 columns); the other dims pass through.
 * inverse != 0 applies the transpose (the reference's BWD variant). */
int ann_op_rope_ht(const void* x, void* y, const float* cs, const float* sn,
                   int32_t B, int32_t T, int32_t H, int32_t D, int32_t pos0,
                   int32_t inverse, int32_t dtype, void* stream);

/* cs, sn (seq_len, head_dim/4) fp32: theta = t * (1/base)^linspace(0,1,D/4). */
int ann_op_rope_tables(float* cs, float* sn, int32_t seq_len, int32_t head_dim,
                       float base, void* stream);

/* y = x * rsqrt(mean(x^2) + eps) over rows of length dim, fp32 math. */
int ann_op_rms_norm(const void* x, void* y, int32_t rows, int32_t dim, float eps,
                    int32_t dtype, void* stream);

/* ---- measurement (no reference counterpart) ------------------------------
 * While enabled, every launch of one kernel class inside the forward calls is
 * bracketed by a HIP event pair recorded on the call's stream (up to
 * max_launches).  ann_profile_read waits for the recorded events and returns
 * the summed duration and the launch count, then clears the record.
 * kind -1 disables. */
#define ANN_PROF_LM_HEAD 0
#define ANN_PROF_QKV 1
#define ANN_PROF_O 2
#define ANN_PROF_FC 3
#define ANN_PROF_PROJ 4
#define ANN_PROF_ATTN 5
#define ANN_PROF_STEP 6   /* the persistent batch-1 decode kernel (whole step) */
int ann_profile_enable(ann_ctx* ctx, int32_t kind, int32_t max_launches);
int ann_profile_read(ann_ctx* ctx, float* total_ms, int32_t* launches);

/* ---- optimizer step (MuonAdam, muon.py:66-137) ----------------------------
 * All arrays are device fp32 unless noted; n elements; outputs may alias the
 * matching inputs.  Scalars as the reference passes them. */
/* adam_step: m' = b1 m + (1-b1) g; v' = b2 v + (1-b2) g^2;
 * u = m' / (sqrt(v') + eps) * step_size; u += p * eff_wd where u * p > 0; p' = p - u. */
int ann_op_adam_step(const float* p, const float* g, const float* m, const float* v, size_t n,
                     float beta1, float beta2, float eps, float step_size, float eff_wd,
                     float* p_out, float* m_out, float* v_out, void* stream);
/* muon_momentum: buf' = buf + (1-mu)(g - buf); geff = g + mu (buf' - g). */
int ann_op_muon_momentum(const float* g, const float* buf, size_t n, float mu, float* geff,
                         float* buf_out, void* stream);
/* muon_apply: p' = p - p*wd*lr (where u*p >= 0) - u*lr. */
int ann_op_muon_apply(const float* p, const float* u, size_t n, float lr, float wd, float* p_out,
                      void* stream);
/* polar_express: g (batch, M, N) fp32 -> out (batch, M, N) bf16, M and N
 * multiples of 64; ws: ann_op_polar_express_ws_bytes(batch, M, N) bytes. */
size_t ann_op_polar_express_ws_bytes(int32_t batch, int32_t M, int32_t N);
int ann_op_polar_express(const float* g, int32_t batch, int32_t M, int32_t N, void* out,
                         void* ws, size_t ws_bytes, void* stream);
/* normuon_rescale: v (batch, M, N) bf16; second_mom (batch, M) if M >= N else
 * (batch, N), updated in place; out (batch, M, N) fp32. */
size_t ann_op_normuon_ws_bytes(int32_t batch, int32_t M, int32_t N);
int ann_op_normuon(const void* v, float* second_mom, int32_t batch, int32_t M, int32_t N,
                   float beta2, float* out, void* ws, size_t ws_bytes, void* stream);

/* NorMuon without an allocation.  No counterpart in the reference: for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight training or serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and results as ann_op_normuon, minus the workspace: the scratch
 * is a fixed device array of ann_op_normuon_noalloc_max_bytes() (4 MiB) inside
 * the library, one per GPU, held until the process ends, so batch * max(M, N)
 * may be at most 524288 (ANN_E_CAPACITY beyond).  The function itself calls
 * no hipMalloc / hipFree.  Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (other streams or threads) race.  The stream
 * must belong to the current device. */
size_t ann_op_normuon_noalloc_max_bytes(void);
int ann_op_normuon_noalloc(const void* v, float* second_mom, int32_t batch, int32_t M, int32_t N,
                           float beta2, float* out, void* stream);

/* Device status of the decode steps (no reference counterpart).  The
 * cross-work-group waits of the persistent batch-1 step and of the decode
 * attention's split combine are bounded; one that gives up sets a device flag
 * and the step's output is not valid.  Synchronises `stream`, returns
 * ANN_E_HIP (and clears the flag) if it is set, else ANN_OK. */
int ann_check_device(ann_ctx* ctx, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* ATTNNN_H */
