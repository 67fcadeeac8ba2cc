// Decode attention: one new token per sequence, QK-norm + RoPE + KV-cache
// append fused in (model.py:244-254).
//
// Grid (nsplit, H, B), 256 threads.  Every work-group of (b, h) first forms
// the new token's q = rope(rms(q)), k = rope(rms(k)) and v from the raw QKV
// projection (one wave, one dim pair per lane), then walks its share of the
// key range [lo, p]: lo = 0 on full-causal layers, p - window + 1 on windowed
// ones.  The key at p itself comes from LDS (this launch is the one writing
// it to the cache; the work-group that owns p stores it for later steps), all
// earlier keys from the cache.
//
// Softmax without a running max: q and k are RMS-normalised rows of Dh
// elements (norm sqrt(Dh) each, up to bf16 rounding), so every score obeys
// |s| <= scale * Dh = shift (host-checked <= 40), and exp(s - shift) lies in
// [e^-2shift, ~1] -- no overflow, no underflow to 0 in fp32.  Splits are then
// plain sums: O_s = sum_j e^(s_j - shift) v_j, L_s = sum_j e^(s_j - shift), and
// o = sum_s O_s / sum_s L_s (rounded once to bf16) is formed by one split of
// (b, h), in split order (deterministic):
//   * every split takes a ticket at its start, one relaxed fetch_add on the
//     (b, h) counter, which only grows: the splits of one launch hold tickets
//     64 r .. 64 r + nsplit - 1 for a round r, and the holder of the last one
//     (ticket % 64 == nsplit - 1) closes the round by adding 64 - nsplit;
//   * each split publishes (O_s, L_s) as tagged words with tag r + 1 (32 bits
//     of data, 32 of tag, one atomic 64-bit store each);
//   * the last ticket holder waits until every split's words carry r + 1 and
//     sums them.  It waits only for splits that already hold a ticket, i.e.
//     have started, so the wait ends whatever the residency of the grid.
// Correctness rests on the RMW order of the counter and on single-word
// coherence, with no fence: no L2 write-back or invalidate at agent scope,
// which measured 10% of a decode step at 16 rows x context 8192.  Counters
// must start at a multiple of 64 (the host clears them before the first
// decode step); the wait is bounded and sets *err if it gives up.
//
// Each wave walks its own 16-key chunks (chunk t of wave w starts at
// k0 + 16 (w + 4 t)) with no work-group barrier inside the loop: 4 lanes x
// Dh/4 dims per key for the scores (bf16 dot2 against the packed q), then
// Dh/8 lanes x 8 dims per V row for P.V; a ring of three chunks is in flight
// per wave.  The four waves' (O, L) are summed once through LDS in wave order.
#include <math.h>
#include <stdlib.h>
#include "common.h"
#include "launch.h"
#include "sk_gemm.h"

namespace ann {

constexpr int AD_THREADS = 256;
constexpr int AD_KW = 16;    // keys per wave chunk

typedef __bf16 ad_bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(ad_bf16x2, a),
                                         __builtin_bit_cast(ad_bf16x2, b), c, false);
}

constexpr int AD_PF_U = 16;   // 16-byte prefetch loads in flight per lane
constexpr unsigned long long AD_PF_MAGIC = 0x9e3779b97f4a7c15ull;

// Prefetch work-group wg of P: reads its share of n16 16-byte words (lanes
// consecutive, AD_PF_U loads in flight) and folds them into one word that is
// stored only if it equals AD_PF_MAGIC.
__device__ __forceinline__ void weight_prefetch(const uint4* __restrict__ p, size_t n16,
                                                unsigned wg, unsigned P,
                                                unsigned long long* __restrict__ sink) {
  const size_t stride = (size_t)P * AD_THREADS;
  uint4 acc = make_uint4(0, 0, 0, 0);
  for (size_t i = (size_t)wg * AD_THREADS + threadIdx.x; i < n16; i += stride * AD_PF_U) {
    uint4 v[AD_PF_U];
#pragma unroll
    for (int u = 0; u < AD_PF_U; ++u) {
      const size_t j = i + u * stride;
      v[u] = j < n16 ? p[j] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < AD_PF_U; ++u) {
      acc.x ^= v[u].x;
      acc.y ^= v[u].y;
      acc.z ^= v[u].z;
      acc.w ^= v[u].w;
    }
  }
  const unsigned long long f = ((unsigned long long)(acc.x ^ acc.z) << 32) | (acc.y ^ acc.w);
  if (f == AD_PF_MAGIC) *sink = f;
}

// The attention of work-group (split, h, b); qkv_src(b, h, t, q, k, v) gives
// lane t's pair of the new token's raw q, k and v.
template <int DH, int RING, typename QKV>
__device__ __forceinline__ void attn_dec_body(
    QKV&& qkv_src, bf16_t* __restrict__ kc, bf16_t* __restrict__ vc,
    const int32_t* __restrict__ pos, const float* __restrict__ cs, const float* __restrict__ sn,
    u64* __restrict__ part, unsigned* __restrict__ cnt, unsigned* __restrict__ err,
    bf16_t* __restrict__ out, int H, int max_ctx, int window, int is_long, float scale, float shift,
    float eps, int nsplit, int split, int h, int b) {
  constexpr int KU = DH / 32;       // 16-byte K slices per lane per chunk (4 lanes per key)
  constexpr int VL = DH / 8;        // lanes per V row
  constexpr int VP = 64 / VL;       // V rows per pass of the wave
  constexpr int VU = AD_KW / VP;    // V passes per chunk (== KU)
  constexpr int P = DH / 2, D4 = DH / 4;

  __shared__ uint32_t s_qp[P];   // q, k of the new token as bf16 pairs
  __shared__ uint32_t s_kp[P];
  __shared__ float s_v[DH];
  __shared__ float s_o[AD_THREADS / 64][DH];
  __shared__ float s_l[AD_THREADS / 64];

  // the wave index as a scalar (the per-chunk test below is uniform)
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the ticket is taken first; its value is read after the barriers below
  __shared__ unsigned s_ticket;
  if (nsplit > 1 && tid == 0)
    s_ticket = __hip_atomic_fetch_add(cnt + b * H + h, 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
  const int d = H * DH;
  const int p = pos[b];
  const int lo = is_long ? 0 : max(0, p - window + 1);
  const int n = p - lo + 1;
  const int per = (n + nsplit - 1) / nsplit;
  const int k0 = lo + split * per;
  const int k1 = min(p + 1, k0 + per);
  const int nch = k1 > k0 ? (k1 - k0 + AD_KW - 1) / AD_KW : 0;
  const int nt = nch > wv ? (nch - wv + 3) / 4 : 0;   // chunks of this wave

  const size_t head_off = ((size_t)b * H + h) * max_ctx;
  const bf16_t* kh = kc + head_off * DH;
  const bf16_t* vh = vc + head_off * DH;
  const int sk = lane >> 2, sd = (lane & 3) * (DH / 4);   // score: key, first dim
  const int vr = lane / VL, vd = (lane % VL) * 8;         // P.V: row in pass, dims

  auto chunk_base = [&](int t) { return k0 + AD_KW * (wv + 4 * t); };
  auto load = [&](int t, uint4* kr, uint4* vr4) {
    const int c = chunk_base(t);
    const int j = c + sk;
    const bool ok = j < k1 && j != p;
#pragma unroll
    for (int u = 0; u < KU; ++u)
      kr[u] = ok ? *(const uint4*)(kh + (size_t)j * DH + sd + u * 8) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < VU; ++u) {
      const int jj = c + vr + u * VP;
      vr4[u] = (jj < k1 && jj != p) ? *(const uint4*)(vh + (size_t)jj * DH + vd)
                                    : make_uint4(0, 0, 0, 0);
    }
  };
  uint4 kb[RING][KU], vb[RING][VU];
#pragma unroll
  for (int r = 0; r < RING - 1; ++r)
    if (r < nt) load(r, kb[r], vb[r]);   // independent of q: overlaps the prologue

  // ---- new token: QK-norm + RoPE (wave 0, one dim pair per lane)
  if (tid < P) {
    uint32_t qw, kw, vw;   // this lane's q, k, v pair of the new token
    qkv_src(b, h, tid, qw, kw, vw);
    float q0 = __uint_as_float(qw << 16), q1 = __uint_as_float(qw & 0xffff0000u);
    float c0 = __uint_as_float(kw << 16), c1 = __uint_as_float(kw & 0xffff0000u);
    const float sq = group_sum<P>(q0 * q0 + q1 * q1);
    const float sk2 = group_sum<P>(c0 * c0 + c1 * c1);
    const float rq = rsqrtf(sq / (float)DH + eps), rk = rsqrtf(sk2 / (float)DH + eps);
    q0 = rbf(q0 * rq); q1 = rbf(q1 * rq);
    c0 = rbf(c0 * rk); c1 = rbf(c1 * rk);
    if (tid < D4) {
      const float c = cs[(size_t)p * D4 + tid], s = sn[(size_t)p * D4 + tid];
      const float a0 = c * q0 + s * q1, a1 = c * q1 - s * q0;
      const float b0 = c * c0 + s * c1, b1 = c * c1 - s * c0;
      q0 = a0; q1 = a1; c0 = b0; c1 = b1;
    }
    s_qp[tid] = pack2(q0, q1);
    const uint32_t kp = pack2(c0, c1);
    s_kp[tid] = kp;
    s_v[2 * tid] = __uint_as_float(vw << 16);
    s_v[2 * tid + 1] = __uint_as_float(vw & 0xffff0000u);
    if (k0 <= p && p < k1) {   // this work-group owns position p: append to the cache
      const size_t ci = (((size_t)b * H + h) * max_ctx + p) * DH + 2 * tid;
      *(uint32_t*)(kc + ci) = kp;
      *(uint32_t*)(vc + ci) = vw;
    }
  }
  __syncthreads();

  uint32_t qp[DH / 8];   // this lane's Dh/4 score dims of q, as pairs
#pragma unroll
  for (int e = 0; e < DH / 8; ++e) qp[e] = s_qp[sd / 2 + e];
  const float sl2 = scale * 1.4426950408889634f, sh2 = shift * 1.4426950408889634f;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  float lsum = 0.f;

  auto compute = [&](int t, const uint4* kr, const uint4* vr4) {
    const int c = chunk_base(t);
    const int j = c + sk;
    // a chunk without the new token (all but at most one per (row, head))
    // takes the score and P.V path without the per-lane tests for it:
    // batch-64 step 0.5498 -> 0.5467 ms, cfg4 0.5026 -> 0.5004 ms.  Not in
    // the register-capped two-chunk ring (cfg5 step 3.055 -> 3.122 ms with it)
    if (RING == 3 && (p < c || p >= c + AD_KW)) {
      float sf = 0.f;
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        sf = dot2_bf16(qp[4 * u + 0], kr[u].x, sf);
        sf = dot2_bf16(qp[4 * u + 1], kr[u].y, sf);
        sf = dot2_bf16(qp[4 * u + 2], kr[u].z, sf);
        sf = dot2_bf16(qp[4 * u + 3], kr[u].w, sf);
      }
      sf += __shfl_xor(sf, 1, 64);
      sf += __shfl_xor(sf, 2, 64);
      const float pf = j < k1 ? __builtin_amdgcn_exp2f(sf * sl2 - sh2) : 0.f;
      if ((lane & 3) == 0) lsum += pf;
#pragma unroll
      for (int u = 0; u < VU; ++u) {
        const float pr = __shfl(pf, 4 * (vr + u * VP), 64);
        float vf[8];
        unpack8(vr4[u], vf);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += pr * vf[e];
      }
      return;
    }
    float s = 0.f;
    if (j == p) {
#pragma unroll
      for (int e = 0; e < DH / 8; ++e) s = dot2_bf16(qp[e], s_kp[sd / 2 + e], s);
    } else {
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        s = dot2_bf16(qp[4 * u + 0], kr[u].x, s);
        s = dot2_bf16(qp[4 * u + 1], kr[u].y, s);
        s = dot2_bf16(qp[4 * u + 2], kr[u].z, s);
        s = dot2_bf16(qp[4 * u + 3], kr[u].w, s);
      }
    }
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    const float pj = j < k1 ? __builtin_amdgcn_exp2f(s * sl2 - sh2) : 0.f;
    if ((lane & 3) == 0) lsum += pj;
#pragma unroll
    for (int u = 0; u < VU; ++u) {
      const int r = vr + u * VP;
      const float pr = __shfl(pj, 4 * r, 64);
      float vf[8];
      if (c + r == p) {
#pragma unroll
        for (int e = 0; e < 8; ++e) vf[e] = s_v[vd + e];
      } else {
        unpack8(vr4[u], vf);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += pr * vf[e];
    }
  };

  for (int t = 0; t < nt; t += RING) {
#pragma unroll
    for (int r = 0; r < RING; ++r) {
      if (t + r < nt) {
        const int tn = t + r + RING - 1;
        if (tn < nt) load(tn, kb[(r + RING - 1) % RING], vb[(r + RING - 1) % RING]);
        compute(t + r, kb[r], vb[r]);
      }
    }
  }

  // ---- (O, L) of this work-group: lanes sharing dims, then waves in order
#pragma unroll
  for (int o = VL; o < 64; o <<= 1)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += __shfl_xor(acc[e], o, 64);
  lsum = group_sum<64>(lsum);
  if (lane < VL) {
#pragma unroll
    for (int e = 0; e < 8; ++e) s_o[wv][vd + e] = acc[e];
  }
  if (lane == 0) s_l[wv] = lsum;
  __syncthreads();
  float ot = 0.f, lt = 0.f;
  if (tid < DH) {
#pragma unroll
    for (int w = 0; w < AD_THREADS / 64; ++w) {
      ot += s_o[w][tid];
      lt += s_l[w];
    }
  }
  if (nsplit == 1) {   // the whole key range: o = O / L
    if (tid < DH) out[(size_t)b * d + h * DH + tid] = f2bf(ot / lt);
    return;
  }
  // partial (O, L) of this split as tagged words; the holder of the round's
  // last ticket sums all of them in split order and writes o = O / L
  const unsigned ticket = s_ticket;
  const uint32_t tag = ticket / 64u + 1u;
  u64* pbase = part + ((size_t)b * H + h) * AD_MAX_SPLIT * (DH + 1);
  u64* pp = pbase + (size_t)split * (DH + 1);
  if (tid < DH) ll_store(pp + tid, __float_as_uint(ot), tag);
  if (tid == 0) ll_store(pp + DH, __float_as_uint(lt), tag);
  if (ticket % 64u != (unsigned)nsplit - 1u) return;
  if (tid == 0)   // close the round: the next launch's tickets start at 64 (r + 1)
    __hip_atomic_fetch_add(cnt + b * H + h, 64u - (unsigned)nsplit, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  if (tid < DH) {
    // up to 8 splits' words loaded at once; the words not yet carrying the
    // tag are re-read together (split order of the sums unchanged)
    float o = 0.f, l = 0.f;
    for (int s0 = 0; s0 < nsplit; s0 += 8) {
      const u64* po[8];
      const u64* pl[8];
      u64 vo[8], vl[8];
      bool ok[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const u64* w = pbase + (size_t)min(s0 + j, nsplit - 1) * (DH + 1);
        ok[j] = s0 + j < nsplit;
        po[j] = w + tid;
        pl[j] = w + DH;
        vo[j] = ll_load(po[j]);
        vl[j] = ll_load(pl[j]);
      }
      ll_settle<8>(po, vo, ok, tag, err);
      ll_settle<8>(pl, vl, ok, tag, err);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (!ok[j]) break;
        o += __uint_as_float((uint32_t)vo[j]);
        l += __uint_as_float((uint32_t)vl[j]);
      }
    }
    out[(size_t)b * d + h * DH + tid] = f2bf(o / l);
  }
}

// RING chunks in flight per wave.  RING 3 takes 195 VGPRs (two work-groups
// per CU); RING 2 is held to 128 (four per CU) for grids of many (b, h)
// work-groups, which then run in fewer rounds.
template <int DH, int RING>
__global__ __launch_bounds__(AD_THREADS) __attribute__((amdgpu_waves_per_eu(RING == 2 ? 3 : 1)))
void k_attn_dec(
    const bf16_t* __restrict__ qkv, bf16_t* __restrict__ kc, bf16_t* __restrict__ vc,
    const int32_t* __restrict__ pos, const float* __restrict__ cs, const float* __restrict__ sn,
    u64* __restrict__ part, unsigned* __restrict__ cnt, unsigned* __restrict__ err,
    bf16_t* __restrict__ out, int H, int max_ctx, int window, int is_long, float scale, float shift,
    float eps, int nsplit, int nb, const uint4* __restrict__ pf, size_t pf_n16,
    unsigned long long* __restrict__ pf_sink) {
  if ((int)blockIdx.z >= nb) {   // grid.z slices past the batch: weight prefetch only
    const unsigned P = (gridDim.z - nb) * gridDim.y * gridDim.x;
    const unsigned wg = ((blockIdx.z - nb) * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
    weight_prefetch(pf, pf_n16, wg, P, pf_sink);
    return;
  }
  const int d = H * DH;
  attn_dec_body<DH, RING>(
      [&](int b, int h, int t, uint32_t& qw, uint32_t& kw, uint32_t& vw) {
        const bf16_t* row = qkv + (size_t)b * 3 * d + h * DH + 2 * t;
        qw = *(const uint32_t*)row;
        kw = *(const uint32_t*)(row + d);
        vw = *(const uint32_t*)(row + 2 * d);
      },
      kc, vc, pos, cs, sn, part, cnt, err, out, H, max_ctx, window, is_long, scale, shift, eps,
      nsplit, blockIdx.x, blockIdx.y, blockIdx.z);
}

// The decode step's RMS + qkv projection and its attention in one launch
// (batch 16..64, d <= 768, direct launches only): work-groups [0, ngemm) run
// the skinny GEMM's 16T x 16T tiles (gemm_sk_body, the same arithmetic as
// k_gemm_sk) and publish bf16 pairs of q, k, v as tagged words xt[m][n / 2]
// (tag = this launch's, from a host counter that only grows); the attention
// work-groups after them (then the weight-prefetch ones) issue their first
// K/V chunks and wait for their (b, h)'s words, so the cache streaming and the
// projection overlap and one launch boundary goes.  Work-groups are
// dispatched in index order, so the projection tiles are resident before any
// attention work-group waits; every wait is bounded.
template <int DH, int RING, int T>
__global__ __launch_bounds__(AD_THREADS) __attribute__((amdgpu_waves_per_eu(RING == 2 ? 3 : 1)))
void k_qkv_attn_dec(
    const bf16_t* __restrict__ x, const bf16_t* __restrict__ wqkv, int ngemm, int gx,
    u64* __restrict__ xt, uint32_t tag, bf16_t* __restrict__ kc, bf16_t* __restrict__ vc,
    const int32_t* __restrict__ pos, const float* __restrict__ cs, const float* __restrict__ sn,
    u64* __restrict__ part, unsigned* __restrict__ cnt, unsigned* __restrict__ err,
    bf16_t* __restrict__ out, int H, int max_ctx, int window, int is_long, float scale, float shift,
    float eps, int nsplit, int nb, const uint4* __restrict__ pf, size_t pf_n16,
    unsigned long long* __restrict__ pf_sink) {
  const int d = H * DH, d2 = d / 2, L = blockIdx.x;
  if (L < ngemm) {
    gemm_sk_body<true, 6, T>(x, d, wqkv, nb, 3 * d, d, eps, L % gx, L / gx,
                             [&](int m, int n, const sk_floatx4_t& v) {
                               float vn[4];
#pragma unroll
                               for (int r = 0; r < 4; ++r) vn[r] = __shfl_down(v[r], 1, 64);
                               if (n & 1) return;
#pragma unroll
                               for (int r = 0; r < 4; ++r)
                                 if (m + r < nb)
                                   ll_store(xt + (size_t)(m + r) * 3 * d2 + (n >> 1),
                                            pack2(v[r], vn[r]), tag);
                             });
    return;
  }
  const int a = L - ngemm, per = nsplit * H;
  if (a >= nb * per) {   // weight prefetch
    weight_prefetch(pf, pf_n16, a - nb * per, gridDim.x - ngemm - nb * per, pf_sink);
    return;
  }
  attn_dec_body<DH, RING>(
      [&](int b, int h, int t, uint32_t& qw, uint32_t& kw, uint32_t& vw) {
        const u64* w = xt + (size_t)b * 3 * d2 + h * (DH / 2) + t;
        qw = ll_wait(w, tag, err);
        kw = ll_wait(w + d2, tag, err);
        vw = ll_wait(w + d, tag, err);
      },
      kc, vc, pos, cs, sn, part, cnt, err, out, H, max_ctx, window, is_long, scale, shift, eps,
      nsplit, a % nsplit, (a / nsplit) % H, a / per);
}

hipError_t qkv_attn_decode(const bf16_t* x, const bf16_t* wqkv, u64* xt, uint32_t tag,
                           bf16_t* kc, bf16_t* vc, const int32_t* pos, const float* cs,
                           const float* sn, u64* part, unsigned* cnt, unsigned* err, bf16_t* out,
                           int B, int H, int Dh, int max_ctx, int window, bool long_layer,
                           float scale, float eps, int nsplit, const WeightPrefetch& pf,
                           hipStream_t st) {
  const int d = H * Dh;
  if (!qkv_attn_fits(B, d, Dh) || nsplit < 1 || nsplit > AD_MAX_SPLIT) return hipErrorInvalidValue;
  const bool pfon = pf.slices > 0 && pf.bytes >= 16 && pf.p && pf.sink;
  if (pfon && ((uintptr_t)pf.p & 15)) return hipErrorInvalidValue;
  const float shift = scale * (float)Dh * 1.02f;
  // the skinny GEMM's tile choice for these shapes (gemm_skinny): 32 x 32
  // tiles above 32 rows (N = 3d >= 2048 here), else 16 x 16
  const int T = B > 32 ? 2 : 1;
  const int gx = (3 * d + 16 * T - 1) / (16 * T), gy = (B + 16 * T - 1) / (16 * T);
  const int ngemm = gx * gy;
  const int natt = nsplit * H * (B + (pfon ? pf.slices : 0));
  const uint4* pfp = pfon ? (const uint4*)pf.p : nullptr;
  const size_t pfn = pfon ? pf.bytes / 16 : 0;
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
  }
  const bool r2 = (long long)nsplit * H * B > 2LL * cus;
#define ANN_QA(R, TT)                                                                          \
  hipLaunchKernelGGL((k_qkv_attn_dec<128, R, TT>), dim3(ngemm + natt), dim3(AD_THREADS), 0, st, \
                     x, wqkv, ngemm, gx, xt, tag, kc, vc, pos, cs, sn, part, cnt, err, out, H,  \
                     max_ctx, window, (int)long_layer, scale, shift, eps, nsplit, B, pfp, pfn,  \
                     pf.sink)
  if (T == 2) {
    if (r2) ANN_QA(2, 2); else ANN_QA(3, 2);
  } else {
    if (r2) ANN_QA(2, 1); else ANN_QA(3, 1);
  }
#undef ANN_QA
  return hipGetLastError();
}

hipError_t attn_decode(const bf16_t* qkv, bf16_t* kc, bf16_t* vc, const int32_t* pos,
                       const float* cs, const float* sn, u64* part, unsigned* cnt, unsigned* err,
                       bf16_t* out,
                       int B, int H, int Dh, int max_ctx, int window, bool long_layer, float scale,
                       float eps, int nsplit, const WeightPrefetch& pf, hipStream_t st) {
  if (nsplit < 1 || nsplit > AD_MAX_SPLIT || B <= 0) return hipErrorInvalidValue;
  const bool pfon = pf.slices > 0 && pf.bytes >= 16 && pf.p && pf.sink;
  if (pfon && ((uintptr_t)pf.p & 15)) return hipErrorInvalidValue;
  const float shift = scale * (float)Dh * 1.02f;
  dim3 grid(nsplit, H, B + (pfon ? pf.slices : 0));
  const uint4* pfp = pfon ? (const uint4*)pf.p : nullptr;
  const size_t pfn = pfon ? pf.bytes / 16 : 0;
  // more than two (b, h, split) work-groups per CU: the three-waves-per-SIMD
  // form (ANN_ATTN_RING=3 / 2 forces one; read at every call)
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
  }
  const char* fe = getenv("ANN_ATTN_RING");
  const int force = fe ? atoi(fe) : 0;
  const bool r2 = force == 2 || (force != 3 && (long long)nsplit * H * B > 2LL * cus);
#define ANN_AD(D, R)                                                                         \
  hipLaunchKernelGGL((k_attn_dec<D, R>), grid, dim3(AD_THREADS), 0, st, qkv, kc, vc, pos, cs, sn, \
                     part, cnt, err, out, H, max_ctx, window, (int)long_layer, scale, shift, eps, \
                     nsplit, B, pfp, pfn, pf.sink)
  switch (Dh) {
    case 64:
      if (r2) ANN_AD(64, 2); else ANN_AD(64, 3);
      break;
    case 128:
      if (r2) ANN_AD(128, 2); else ANN_AD(128, 3);
      break;
    default:
      return hipErrorInvalidValue;
  }
#undef ANN_AD
  return hipGetLastError();
}

}  // namespace ann
