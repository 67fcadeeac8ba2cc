// Host-side launchers of the gfx950 kernels (internal to libattnnn.so).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "common.h"

namespace ann {

// Epilogue of a projection y = a @ W^T (W stored (N, K)):
//   EPI_STORE       out = bf16(y)
//   EPI_RELU2       out = bf16(max(bf16(y), 0)^2)                 (model.py:258)
//   EPI_RESID_ATTN  x = ((r0*x) + (p0*bf16(y))) + (x0l*x0), each op
//                   rounded to bf16                               (model.py:255-256)
//   EPI_RESID_MLP   x = (r1*x) + (p1*bf16(y)), each op rounded     (model.py:259-260)
//   EPI_LOGITS      z = bf16(y) -> zbuf (if set); softcap(z) -> logits fp32 (if set)
//   EPI_QKV         (MFMA GEMM only, prefill QKV projection) per head:
//                   q = rope(rms(bf16(y_q))) -> out (M, ldo); k = rope(rms(bf16(y_k)))
//                   and v = bf16(y_v) -> the KV cache at [b][h][pos[b] + t]
//                   (model.py:244-247, 252)
//   EPI_CE          (MFMA GEMM only, lm_head of the training forward) per row m and
//                   128-column tile t: ce_part[t * ldz + m] = sum of exp(softcap(bf16(y)))
//                   over the tile's columns; ce_tz[m] = softcap(bf16(y[tgt[m]])) from
//                   the tile holding the target (metal_kernels.py:153-193)
//   EPI_TOPK        (MFMA GEMM only, decode lm_head of 3..511 rows) per row m and
//                   128-column tile t, over the columns n < Vs: the tile's 8
//                   largest words (zkey(bf16(y)) << 16 | 0xffff - n, so equal
//                   keys rank the lower column first) to cand[(m nt + t) 8 ..],
//                   largest first (0 past the valid columns), and its 9th
//                   largest word to cand_r[m nt + t]; softcap(z) -> logits fp32
//                   (if set).  No z is stored (sample.py:44-49 via sample_cand)
//   EPI_PE_B        (Polar Express) out = bf16(bf16(s0*x) + bf16(s1*bf16(y)))  (muon.py:37)
//   EPI_PE_X        (Polar Express) out = bf16(bf16(s0*x) + bf16(y))           (muon.py:38,42)
//                   x is the epilogue's second operand (M, ldr); when outT is set
//                   the same values also go to outT (N, ldoT), transposed
enum { EPI_STORE = 0, EPI_RELU2 = 1, EPI_RESID_ATTN = 2, EPI_RESID_MLP = 3, EPI_LOGITS = 4,
       EPI_QKV = 5, EPI_CE = 6, EPI_PE_B = 7, EPI_PE_X = 8, EPI_TOPK = 9 };

// Candidates a 128-column lm_head tile emits per row (EPI_TOPK).
constexpr int TK_M = 8;

struct EpiArgs {
  bf16_t* out;       // STORE / RELU2 output (M, ldo)
  int ldo;
  bf16_t* x;         // residual stream (M, ldr), updated in place
  const bf16_t* x0;  // x0 (M, ldr)
  int ldr;
  const float* lam;  // this layer's lambda row: r0 r1 p0 p1 x0l
  bf16_t* z;         // LOGITS: bf16 z (M, ldz) or null
  float* logits;     // LOGITS: fp32 softcapped (M, ldz) or null
  int ldz;
  // LOGITS + greedy (GEMV only): each work-group stores its best packed key
  // (ordered z << 32 | ~n, over columns n < Vs) per row to
  // amax[m * blocks + block]; argmax_finalize turns them into tokens.
  unsigned long long* amax;
  int Vs;
  // TOPK: candidate words (M, nt, TK_M) and 9th-largest words (M, nt);
  // tk_first: greedy rows, only each tile's largest word (cand[.. * TK_M])
  uint32_t* cand;
  uint32_t* cand_r;
  int nt, tk_first;
  // QKV: row m = b * T + t; model dim d = H * Dh; caches [B][H][max_ctx][Dh]
  bf16_t* kc;
  bf16_t* vc;
  const int32_t* pos;
  const float* cs;   // RoPE cos / sin tables (max_ctx, Dh / 4)
  const float* sn;
  int T, H, Dh, max_ctx;
  float eps;
  // CE: per-tile partial sums (ldz = row stride of a tile's slice), target
  // logits, targets
  float* ce_part;
  float* ce_tz;
  const int32_t* tgt;
  // PE_B / PE_X scalars
  float s0, s1;
  // PE_X: transposed copy of the output, or null
  bf16_t* outT;
  int ldoT;
  // batched STORE / PE_B with a symmetric M x M output (x x^T, b A + c A A):
  // only the tiles on and above the diagonal are computed, each one above it
  // also stored transposed at the mirrored position
  int sym;
};

// Sampling parameters read by the sampler from device memory (so a captured
// decode step replays with new values); step[b] counts draws per sequence.
struct SampParams {
  float temperature;
  int top_k;
  unsigned long long seed;
};

// Input prologue of a projection: X rows as given or RMS-normalised.
enum { PRE_PLAIN = 0, PRE_RMS = 1 };

hipError_t pack_transpose(const float* src, bf16_t* dst, int K, int N, int ldd,
                          const float* scale, hipStream_t st);
hipError_t pack_cast(const float* src, bf16_t* dst, size_t n, hipStream_t st);
hipError_t pack_lambdas(const float* resid, const float* post, const float* x0l, float* out,
                        int L, hipStream_t st);
hipError_t rope_tables(float* cs, float* sn, int seq_len, int head_dim, float base,
                       hipStream_t st);
hipError_t embed_rms(const int32_t* tok, const bf16_t* emb, bf16_t* x, bf16_t* x0, int M, int d,
                     int V, float eps, hipStream_t st);
hipError_t qkv_post(const bf16_t* qkv, bf16_t* q, bf16_t* kc, bf16_t* vc, const int32_t* pos,
                    const float* cs, const float* sn, int M, int T, int H, int Dh, int max_ctx,
                    float eps, hipStream_t st);

// GEMV for M <= 8 rows: y = pre(X) @ W^T, X (M, ldx) bf16.
hipError_t gemv(int epi, int pre, const bf16_t* W, const bf16_t* X, int ldx, int M, int N, int K,
                float eps, const EpiArgs& ea, hipStream_t st);
bool gemv_fits(int M, int K);
bool gemv_routes(int M, int K);   // the engine's choice: the rows the GEMV takes
int gemv_blocks(int N, int K);
hipError_t argmax_finalize(const unsigned long long* keys, int nkeys, int M, int32_t* out_tok,
                           int32_t* pos, int pos_adv, hipStream_t st);
// Skinny MFMA GEMM for decode (M <= 128, K % 128 == 0): y = pre(A) @ W^T,
// rms: A rows RMS-normalised in the kernel (K <= 3072).
bool gemm_skinny_fits(int M, int N, int K, bool rms);
bool gemm_qkv_fits(int M, int N, int K, const EpiArgs& ea);
// k_gemm over `batch` independent problems (blockIdx.z); epilogues STORE,
// PE_B, PE_X; sOut / sX are the batch strides of ea.out / ea.x.
// Large projections (prefill, training forward): 256 x 256 tiles, one work-
// group per CU, AGPR accumulators, staged 16-byte epilogues.  Takes EPI_STORE,
// EPI_RELU2, EPI_RESID_ATTN, EPI_RESID_MLP and EPI_QKV; gemm_big_fits says
// whether a shape can go there, gemm_big_routes which epilogues gemm() sends
// there by itself (those measured faster than the k_gemm_2w tiles).
bool gemm_big_fits(int epi, const bf16_t* A, int lda, int M, int N, int K, const EpiArgs& ea);
bool gemm_big_routes(int epi, int M, int N);
hipError_t gemm_big(int epi, const bf16_t* A, int lda, const bf16_t* W, int M, int N, int K,
                    const EpiArgs& ea, hipStream_t st);
hipError_t gemm_batched(int epi, const bf16_t* A, int lda, long long sA, const bf16_t* W,
                        long long sW, int M, int N, int K, const EpiArgs& ea, long long sOut,
                        long long sX, int batch, hipStream_t st);
// Optimizer step (optim.hip).
hipError_t adam_step(const float* p, const float* g, const float* m, const float* v, size_t n,
                     float b1, float b2, float eps, float step, float wd, float* po, float* mo,
                     float* vo, hipStream_t st);
hipError_t muon_momentum(const float* g, const float* buf, size_t n, float mu, float* geff,
                         float* bo, hipStream_t st);
hipError_t muon_apply(const float* p, const float* u, size_t n, float lr, float wd, float* po,
                      hipStream_t st);
size_t polar_express_ws_bytes(int batch, int M, int N);
hipError_t polar_express(const float* g, int batch, int M, int N, bf16_t* out, void* ws,
                         size_t ws_bytes, hipStream_t st);
size_t normuon_ws_bytes(int batch, int M, int N);
hipError_t normuon(const bf16_t* v, float* second_mom, int batch, int M, int N, float beta2,
                   float* out, void* ws, size_t ws_bytes, hipStream_t st);
// NorMuon with its scratch in a fixed device array of NM_SCRATCH_BYTES (no
// allocation; calls that overlap on one GPU race); normuon_ws_bytes(batch, M,
// N) must not exceed it.
constexpr size_t NM_SCRATCH_BYTES = (size_t)4 << 20;
hipError_t normuon_noalloc(const bf16_t* v, float* second_mom, int batch, int M, int N,
                           float beta2, float* out, hipStream_t st);
// Per-row loss = log(sum over tiles of ce_part) - ce_tz (tiles summed in
// order), written to rows[M]; mean over the rows (fixed order) to *mean.
hipError_t ce_finalize(const float* part, int ld, int ntiles, const float* tz, int M, float* rows,
                       float* mean, hipStream_t st);
hipError_t gemm_skinny(int epi, bool rms, const bf16_t* A, int lda, const bf16_t* W, int M, int N,
                       int K, float eps, const EpiArgs& ea, hipStream_t st);
hipError_t gemm_decode64(int epi, const bf16_t* A, int lda, const bf16_t* W, int M, int N, int K,
                         const EpiArgs& ea, hipStream_t st);
// MFMA GEMM (prefill): y = A @ W^T with A (M, lda) bf16.
hipError_t gemm(int epi, const bf16_t* A, int lda, const bf16_t* W, int M, int N, int K,
                const EpiArgs& ea, hipStream_t st);
// h = bf16(rms(x)) for M rows of length d (row strides ldx / ldh).
hipError_t rms_apply(const bf16_t* x, int ldx, bf16_t* h, int ldh, int M, int d, float eps,
                     hipStream_t st);

// Prefill attention (MFMA flash attention) of B x T query rows at positions
// pos[b] + t against keys [window start, own position] of the cache.
hipError_t attn_prefill(const bf16_t* q, const bf16_t* kc, const bf16_t* vc, const int32_t* pos,
                        bf16_t* out, int B, int T, int H, int Dh, int max_ctx, int window,
                        bool long_layer, float scale, hipStream_t st);

// Weights read ahead by extra work-groups of a decode attention launch, so
// that the projections after it find them in the memory-side cache instead
// of HBM.  slices = extra grid.z slices (each nsplit x H work-groups); 0 = none.
// sink: one 8-byte word the reads are folded into (written only on a 64-bit
// match with a fixed constant, so the loads cannot be optimised away).
constexpr int AD_MAX_SPLIT = 32;   // key splits per (b, h) of the decode attention

struct WeightPrefetch {
  const void* p = nullptr;   // 16-byte aligned
  size_t bytes = 0;
  int slices = 0;
  unsigned long long* sink = nullptr;
};

// Decode attention with fused QK-norm / RoPE / KV append (one token per
// sequence) -> out (B, H*Dh) bf16.  part: split scratch of tagged words
// (B, H, AD_MAX_SPLIT, Dh + 1) -- a fixed stride per (b, h), so a slot is only
// ever written by the splits of its own (b, h), whose tags only grow, whatever
// nsplit a launch uses; cnt: B*H ticket counters, multiples of 64 between
// calls (zero before the first, with part zeroed too); err: set if a bounded
// wait gave up.
hipError_t attn_decode(const bf16_t* qkv, bf16_t* kc, bf16_t* vc, const int32_t* pos,
                       const float* cs, const float* sn, u64* part, unsigned* cnt, unsigned* err,
                       bf16_t* out,
                       int B, int H, int Dh, int max_ctx, int window, bool long_layer, float scale,
                       float eps, int nsplit, const WeightPrefetch& pf, hipStream_t st);
// The decode step's RMS + qkv projection (x (B, d) against wqkv (3d, d)) and
// the attention above in one launch: q, k, v handed over as tagged words in
// xt (B x 3d/2 words; `tag` larger than any earlier launch's on that buffer).
// Shapes it takes: 16..64 rows, Dh 128, d a multiple of 128 up to 768.
constexpr bool qkv_attn_fits(int B, int d, int Dh) {
  return B >= 16 && B <= 64 && Dh == 128 && d % 128 == 0 && d <= 768;
}
hipError_t qkv_attn_decode(const bf16_t* x, const bf16_t* wqkv, u64* xt, uint32_t tag,
                           bf16_t* kc, bf16_t* vc, const int32_t* pos, const float* cs,
                           const float* sn, u64* part, unsigned* cnt, unsigned* err, bf16_t* out,
                           int B, int H, int Dh, int max_ctx, int window, bool long_layer,
                           float scale, float eps, int nsplit, const WeightPrefetch& pf,
                           hipStream_t st);

// Sampling of B rows of bf16 z (B, ldz) over the first Vs entries with the
// device-resident parameters; uses and increments steps[b]; advances pos[b]
// by pos_adv.
hipError_t sample(const bf16_t* z, int ldz, int B, int Vs, const SampParams* sp,
                  unsigned long long* steps, int32_t* out_tok, int32_t* pos, int pos_adv,
                  hipStream_t st);
// One-time set-up of the candidate sampler (its dynamic LDS limit), called by
// the entry points before anything they may capture into a graph.
hipError_t sample_prepare();
// The same draw from top-k candidates instead of z: B rows of nt tiles
// (holders of them with valid columns), per tile its TK_M largest words
// (zkey << 16 | 0xffff - n) in cand (B, nt, TK_M) and its next word in
// cand_r (B, nt).  Where the candidates cannot prove the kept set complete
// (ties or clusters beyond TK_M keys in a tile, top_k 0 or above the tiles)
// the row is sampled whole: from z (B, N) when the producer stored it (the
// persistent step), else from the 128-column lm_head tiles concerned,
// recomputed from A (the lm_head's normalised input rows, lda) and W (N x K)
// with the GEMM's MFMA sequence (bit-identical z).  verify (null normally,
// recompute form only): recompute every tile and set bit 1 of *verify where
// a tile's top TK_M + 1 words differ from the candidates.
hipError_t sample_cand(const uint32_t* cand, const uint32_t* cand_r, int nt, int holders, int B,
                       int Vs, const bf16_t* z, const bf16_t* A, int lda, const bf16_t* W, int N,
                       int K, const SampParams* sp, unsigned long long* steps, int32_t* out_tok,
                       int32_t* pos, int pos_adv, unsigned* verify, hipStream_t st);
hipError_t set_sampling(SampParams* sp, unsigned long long* steps, int B, float temperature,
                        int top_k, unsigned long long seed, unsigned long long step,
                        hipStream_t st);
hipError_t set_pos(int32_t* pos, int B, int value, hipStream_t st);
hipError_t advance_pos(int32_t* pos, int B, int n, hipStream_t st);

// Persistent decode step (1 .. PD_MAX_B rows): one launch of G work-groups
// (one per CU, all resident) runs embed, all layers, lm_head and (greedy) the
// argmax; see decode_persist.hip.  Exchange words are 64-bit (tag << 32 | data).
typedef unsigned long long u64;
struct PDParams {
  const bf16_t* emb;
  const bf16_t* head;
  const bf16_t* layers;   // layer 0; layer l at layers + l * lstride
  size_t lstride, o_qkv, o_o, o_fc, o_proj;   // elements
  const float* lam;       // (L, 8): r0 r1 p0 p1 x0l
  const float* cs;
  const float* sn;
  bf16_t* kc;             // caches of layer 0; layer l at + l * kvl
  bf16_t* vc;
  size_t kvl;
  u64 long_mask;
  const int32_t* tok;
  int32_t* out_tok;
  int32_t* pos;
  bf16_t* z;              // !greedy: bf16 logits (B, V)
  float* logits;          // optional fp32 softcapped logits (B, V)
  u64* xq;                // qkv       B x 3d/2 words
  u64* xp;                // partials  PD_REP_P copies of B*H*s_long x (Dh+1), p_stride apart
  u64* xm;                // x'        rep copies of B x d/2, rep_stride words apart
  u64* xh;                // hidden    PD_REP_H copies of B x 2d, h_stride words apart
  u64* xx;                // x         rep copies of B x d/2, rep_stride words apart
  u64* xk;                // keys      G x B
  unsigned* gen;          // step generation (tags)
  unsigned* err;          // set when a bounded wait timed out
  int d, H, L, V, Vs, max_ctx, window, s_win, s_long, greedy;
  int rep, rep_stride;    // copies of xm / xx (1..PD_MAX_REP); work-group g reads copy g % rep
  int h_stride;           // xh: PD_REP_H copies, work-group g reads copy g % PD_REP_H
  int p_stride;           // xp: PD_REP_P copies, work-group g reads copy g % PD_REP_P
  int on;                 // work-groups holding the o rows (at most, after the attention ones)
  float scale, shift, eps;
  // !greedy (or null): per row and work-group the TK_M largest words of its
  // z slice and the next one (sample_cand's tiles: the G row slices).  Last
  // in the struct: placed after z they moved the fields behind them and the
  // 155M batch-1 greedy step measured 1.1% slower
  uint32_t* cand;
  uint32_t* cand_r;
  // one row: each head's qkv rows and attention splits on XCD h (see
  // decode_persist_xcd_ok), else contiguous over the work-groups
  int head_xcd;
};
constexpr int PD_MAX_REP = 8;
// Copies of the h and attention-partial exchanges (their areas hold up to
// PD_MAX_REP).  Fewer pollers per copy: the 155M batch-1 generation 181.4 ->
// 178.8 and 178.4 -> 176.8 ms (two boxes, alternating A/B) with 4 of each
// against one; 8 h / 4 partial copies 179.9.  Compile-time counts: the same
// copies chosen at run time measured 6% slower (loops and modulo in the step).
constexpr int PD_REP_H = 4, PD_REP_P = 4;
constexpr int PD_MAX_B = 4;                       // rows of the persistent step
// lm_head rows per lane of the persistent step's top-k candidates: a
// work-group's vocabulary slice of at most 64 PD_ZE rows
constexpr int PD_ZE = 8;
constexpr size_t PD_MAX_LDS = (size_t)144 * 1024; // its dynamic LDS (row buffers + partials)
constexpr int PD_MAX_SLONG = 8;                   // attention splits per (row, head)
constexpr int PD_MAX_G = 1024;                    // work-groups

// Exchange area of the persistent decode step (up to PD_MAX_B rows): 64-bit
// tagged words of xq, xp, xm, xh, xx, xk, then the generation and error
// words (strides in words, pd_layout offsets in bytes).  xm and xx hold
// PD_MAX_REP copies pd_rep_stride words apart; xp and xh have room for PD_MAX_REP copies pd_p_stride / pd_h_stride
// apart, of which the step uses PD_REP_P / PD_REP_H (the measured layout:
// packing the areas tighter moved the step's time by up to 2.7%).  Functions
// of d and H only, so a kernel instance with both as constants derives every
// area from xq at compile time.
constexpr size_t pd_round64(size_t v) { return (v + 63) / 64 * 64; }
constexpr size_t pd_rep_stride(size_t d) { return pd_round64((size_t)PD_MAX_B * d / 2); }
constexpr size_t pd_h_stride(size_t d) { return pd_round64((size_t)PD_MAX_B * 2 * d); }
constexpr size_t pd_p_stride(size_t d, size_t H) {
  return pd_round64((size_t)PD_MAX_B * H * PD_MAX_SLONG * (d / H + 1));
}
// Byte offset of part `which` (1..8) from the area's start (256-byte aligned
// parts), 0: the total size.
constexpr size_t pd_layout(size_t d, size_t H, int which) {
  const size_t B = PD_MAX_B, rs = pd_rep_stride(d);
  const size_t parts[8] = {B * 3 * d / 2,        PD_MAX_REP * pd_p_stride(d, H),
                           PD_MAX_REP * rs,        PD_MAX_REP * pd_h_stride(d),
                           PD_MAX_REP * rs,        (size_t)PD_MAX_G * B,
                           1,                      1};
  size_t off = 0;
  for (int i = 0; i < 8; ++i) {
    if (which == i + 1) return off;
    off += (parts[i] * 8 + 255) / 256 * 256;
  }
  return off;
}
bool decode_persist_fits(int B, int d, int H, int Dh, int V, int L, int G, int s_long);
bool decode_persist_xcd_ok(int B, int d, int H, int Dh, int G, int s_long);
size_t decode_persist_lds(int B, int d, int H, int Dh, int s_long);
// specialize: take the compile-time instance of a model shape that has one
// (155M at 1-4 rows), else the generic kernel
hipError_t decode_persist(const PDParams& P, int B, int Dh, int G, bool coop, bool specialize,
                          hipStream_t st);

hipError_t op_relu2(const void* x, void* y, size_t n, int dtype, hipStream_t st);
hipError_t op_rope(const void* x, void* y, const float* cs, const float* sn, int B, int T, int H,
                   int D, int pos0, int inverse, int dtype, hipStream_t st);
hipError_t op_rms(const void* x, void* y, int rows, int dim, float eps, int dtype, hipStream_t st);

}  // namespace ann
