// Persistent decode step for 1 to 4 rows (BM): embed, every layer, lm_head
// and the greedy argmax of one token per row in ONE launch of G 512-thread
// work-groups, at most one per CU, all resident at once (model.py:223-263 for
// T = 1, sample.py:44-49 greedy).  The host picks G (3/4 of the CUs where the
// rows fit: fewer work-groups exchange faster, measured).  Every projection
// row's weights are read once per step and applied to the BM rows held in
// LDS; the attention runs one work-group per (row, head, split).
//
// Why: at batch 1 a decode step is ~57 dependent phases whose own work is a
// few microseconds of weight streaming; as separate kernels every phase pays
// a launch and a cold memory round trip.  Here the work-groups stay resident
// and hand the small activation vectors to each other through LL exchanges:
// every 64-bit word carries 32 bits of data and a 32-bit tag (step
// generation * 256 + phase), written with one relaxed device-scope store and
// polled with device-scope loads -- data and "ready" arrive together, no
// fence and no barrier.  Each phase issues its weight (and K/V) loads before
// it waits for its input, so their latency hides behind the exchange.
//
// Phases of layer l (tags 5l+1 .. 5l+5), rows of every projection split over
// all work-groups in pairs (one tagged word = two bf16 outputs):
//   1  qkv  = rms(x) Wqkv^T                       -> xq
//   2  attention of (head h, split s): QK-norm, RoPE, cache append, softmax
//      partial (O, L) with a fixed shift (|s| <= scale Dh) -> xp
//   3  o = sum_s O_s / sum_s L_s; x' = mix_attn(x, x0, o Wo^T)  -> xm
//      (rows on the work-groups that ran no attention in phase 2)
//   4  h = relu2(rms(x') Wfc^T)                   -> xh
//   5  x = mix_mlp(x', h Wproj^T)                 -> xx
// then z = rms(x) lm_head^T: greedy keys (bf16 order << 16 | 0xffff - n) per
// work-group -> xk, work-group 0 picks the token and advances pos; otherwise
// z is stored for the sampler kernel.
//
// Every wait is bounded: after LL_SPIN polls (or once any work-group has
// flagged a timeout in *err) it gives up and the kernel runs to its end, so
// all waves always exit; the host reports a set flag as an error.  The grid
// must be co-resident: G <= the CU count, a CU holds one (see pd_launch).
#include <math.h>
#include "common.h"
#include "launch.h"

namespace ann {

constexpr int PD_T = 512;
constexpr int PD_NW = PD_T / 64;
constexpr int PD_SLOTS = 12;                 // 16-byte weight chunks per lane in flight
constexpr int PD_RMAX = PD_NW * PD_SLOTS;    // projection rows per work-group (U = 1)
extern "C" __device__ unsigned __ockl_wfred_max_u32(unsigned);
constexpr int PD_KW = 16;                    // keys per wave chunk
constexpr uint32_t PD_PH = 256;              // tags per step

typedef __bf16 pd_bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float pd_dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(pd_bf16x2, a),
                                         __builtin_bit_cast(pd_bf16x2, b), c, false);
}
__device__ __forceinline__ float pd_dot8(const uint4& w, const uint4& x, float c) {
  c = pd_dot2(w.x, x.x, c);
  c = pd_dot2(w.y, x.y, c);
  c = pd_dot2(w.z, x.z, c);
  return pd_dot2(w.w, x.w, c);
}

// dst[i] = data of src[i] for i < n (n >= 1): up to 8 words per thread read
// at once, then the ones not yet tagged re-read together.  Slots past n load
// nothing (a clamped address would have every work-group poll the last word
// up to 7 more times per thread, measured slower).
__device__ __forceinline__ void ll_poll(const u64* src, int n, uint32_t* dst, uint32_t tag,
                                        unsigned* err) {
  for (int i0 = 0; i0 < n; i0 += PD_T * 8) {
    const u64* p[8];
    u64 v[8];
    bool ok[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = i0 + j * PD_T + (int)threadIdx.x;
      ok[j] = i < n;
      p[j] = src + min(i, n - 1);
      v[j] = ok[j] ? ll_load(p[j]) : 0ull;
    }
    ll_settle<8>(p, v, ok, tag, err);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = i0 + j * PD_T + (int)threadIdx.x;
      if (ok[j]) dst[i] = (uint32_t)v[j];
    }
  }
}

// The K = d projections (qkv, o, fc) give each wave up to PD_PW pairs of
// consecutive rows (PD_PW * 2 * UD weight chunks per lane in registers), so
// a wave forms its own bf16 pairs and stores them without LDS staging or a
// barrier; the K = 4d projection holds one row of 4 UD chunks per wave.
constexpr int PD_PW = 2;

// Rows of a projection owned by work-group g: pairs [b, e) of npairs, split
// over the `count` work-groups from `first` on (none for the others).
__device__ __forceinline__ void pd_rows_at(int npairs, int& n0, int& nr, int g, int G) {
  if (g < 0 || g >= G) {
    n0 = nr = 0;
    return;
  }
  const int b = (int)((long long)npairs * g / G), e = (int)((long long)npairs * (g + 1) / G);
  n0 = 2 * b;
  nr = 2 * (e - b);
}
__device__ __forceinline__ void pd_rows(int npairs, int& n0, int& nr, int first, int count) {
  pd_rows_at(npairs, n0, nr, (int)blockIdx.x - first, count);
}

// qkv rows of work-group g.  With xcd (one row, H <= 8, shares checked by
// decode_persist_xcd_ok) the q, k and v rows of head h come from the
// work-groups of XCD h (work-group g runs on XCD g % 8), which also run that
// head's attention splits, so that hand-off stays inside one XCD: the 3 Dh/2
// row pairs of the head split evenly over the XCD's G / 8 work-groups, each
// share inside its q, k or v rows.  XCDs numbered H and up hold none.
// Otherwise the pairs split contiguously over all work-groups.
template <int P2>
__device__ __forceinline__ void pd_rows_qkv(int xcd, int H, int d2, int& n0, int& nr) {
  if (!xcd) {
    pd_rows(3 * d2, n0, nr, 0, (int)gridDim.x);
    return;
  }
  const int g = (int)blockIdx.x, x = g & 7, i = g >> 3, per = (int)gridDim.x >> 3;
  if (x >= H) {
    n0 = nr = 0;
    return;
  }
  const int b = 3 * P2 * i / per, e = 3 * P2 * (i + 1) / per;
  const int part = b / P2;   // 0 q, 1 k, 2 v
  n0 = 2 * (part * d2 + x * P2 + (b - part * P2));
  nr = 2 * (e - b);
}

// Attention unit (b * H + h) * S + s run by work-group g, or -1.  xcd (one
// row): unit (h, s) on work-group 8 s + h, i.e. on XCD h with the head's qkv
// rows; otherwise units 0 .. NA - 1 on work-groups 0 .. NA - 1.
__device__ __forceinline__ int pd_attn_unit(int xcd, int g, int H, int S, int NA) {
  if (!xcd) return g < NA ? g : -1;
  const int x = g & 7, q = g >> 3;
  return x < H && q < S ? x * S + q : -1;
}

// Index of work-group g among those without an attention unit (the o rows
// go to the first of them).
__device__ __forceinline__ int pd_free_index(int xcd, int g, int H, int S, int NA) {
  if (!xcd) return g - NA;
  const int x = g & 7, q = g >> 3;
  return g - (q < S ? q * H + min(x, H) : S * H);
}

// Weight chunks of this lane: row n0 + wave + 8 rr (rr < R), chunks
// lane + 64 u (u < U).
template <int U, int R>
__device__ __forceinline__ void pd_wload(const bf16_t* W, int K, int n0, int nr, uint4* wr) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, K8 = K >> 3;
#pragma unroll
  for (int rr = 0; rr < R; ++rr) {
    const int r = wv + PD_NW * rr;
    const bool ok = r < nr;
    const uint4* row = (const uint4*)(W + (size_t)(n0 + (ok ? r : 0)) * K);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = lane + 64 * u;
      wr[rr * U + u] = (ok && c < K8) ? row[c] : make_uint4(0u, 0u, 0u, 0u);
    }
  }
}

// stage[b][r] = dot(row r, gin[b]) for the nr rows of this work-group.
template <int U, int R, int BM>
__device__ __forceinline__ void pd_wdot(const uint4* wr, const uint4* gin, int K, int nr,
                                        float (*stage)[PD_RMAX]) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, K8 = K >> 3;
#pragma unroll
  for (int rr = 0; rr < R; ++rr) {
    const int r = wv + PD_NW * rr;
    if (r < nr) {
      float acc[BM];
#pragma unroll
      for (int b = 0; b < BM; ++b) acc[b] = 0.f;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = lane + 64 * u;
        if (c < K8) {
#pragma unroll
          for (int b = 0; b < BM; ++b) acc[b] = pd_dot8(wr[rr * U + u], gin[b * K8 + c], acc[b]);
        }
      }
#pragma unroll
      for (int b = 0; b < BM; ++b) {
        const float t = wave_sum(acc[b]);
        if (lane == 0) stage[b][r] = t;
      }
    }
  }
  __syncthreads();
}

// dst = bf16(src * rsqrt(mean(src^2) + eps)) for BM rows of K (LDS to LDS).
template <int BM>
__device__ __forceinline__ void pd_rms(const bf16_t* src, bf16_t* dst, int K, float eps,
                                       float (*red)[PD_NW]) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint32_t* s2 = (const uint32_t*)src;
  uint32_t* d2 = (uint32_t*)dst;
  const int K2 = K >> 1;
  float sc[BM];
#pragma unroll
  for (int b = 0; b < BM; ++b) {
    float ss = 0.f;
    for (int i = tid; i < K2; i += PD_T) {
      const uint32_t w = s2[b * K2 + i];
      const float a = __uint_as_float(w << 16), c = __uint_as_float(w & 0xffff0000u);
      ss += a * a + c * c;
    }
    ss = wave_sum(ss);
    if (lane == 0) red[b][wv] = ss;
  }
  __syncthreads();
#pragma unroll
  for (int b = 0; b < BM; ++b) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < PD_NW; ++w) t += red[b][w];
    sc[b] = rsqrtf(t / (float)K + eps);
  }
#pragma unroll
  for (int b = 0; b < BM; ++b)
    for (int i = tid; i < K2; i += PD_T) {
      const uint32_t w = s2[b * K2 + i];
      d2[b * K2 + i] = pack2(__uint_as_float(w << 16) * sc[b], __uint_as_float(w & 0xffff0000u) * sc[b]);
    }
  __syncthreads();
}

enum { PE_STORE = 0, PE_ATTN = 1, PE_RELU2 = 2, PE_MLP = 3 };

// Epilogue of outputs n, n + 1 of row b: the bf16 pair of one tagged word.
template <int E>
__device__ __forceinline__ uint32_t pd_epi(float y0, float y1, int b, int n, const float* lam,
                                           const bf16_t* xr, const bf16_t* x0, int d) {
  if (E == PE_STORE) return pack2(y0, y1);
  if (E == PE_RELU2) return (uint32_t)relu2_bf(y0) | ((uint32_t)relu2_bf(y1) << 16);
  if (E == PE_ATTN) {
    const bf16_t a = mix_attn(lam, bf2f(xr[b * d + n]), bf2f(x0[b * d + n]), y0);
    const bf16_t c = mix_attn(lam, bf2f(xr[b * d + n + 1]), bf2f(x0[b * d + n + 1]), y1);
    return (uint32_t)a | ((uint32_t)c << 16);
  }
  const bf16_t a = mix_mlp(lam, bf2f(xr[b * d + n]), y0);
  const bf16_t c = mix_mlp(lam, bf2f(xr[b * d + n + 1]), y1);
  return (uint32_t)a | ((uint32_t)c << 16);
}

// Weight chunks of this lane for the pair path: pairs q = wave + NW k
// (k < PD_PW), rows 2q and 2q + 1 of [n0, n0 + nr), chunks lane + 64 u.
template <int U>
__device__ __forceinline__ void pd_wload2(const bf16_t* W, int K, int n0, int nr, uint4* wr) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, K8 = K >> 3;
#pragma unroll
  for (int k = 0; k < PD_PW; ++k) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = 2 * (wv + PD_NW * k) + h;
      const bool ok = r < nr;
      const uint4* row = (const uint4*)(W + (size_t)(n0 + (ok ? r : 0)) * K);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = lane + 64 * u;
        wr[(2 * k + h) * U + u] = (ok && c < K8) ? row[c] : make_uint4(0u, 0u, 0u, 0u);
      }
    }
  }
}

// Dots of this wave's pairs with gin, epilogue, and the tagged stores of the
// pairs to dst (row stride rw words) and its rep copies cst words apart --
// per wave, as soon as its own sums are done.
template <int E, int U, int BM>
__device__ __forceinline__ void pd_wdot2(const uint4* wr, const uint4* gin, int K, int n0, int nr,
                                         u64* dst, int rw, uint32_t tag, const float* lam,
                                         const bf16_t* xr, const bf16_t* x0, int d, int rep,
                                         int cst) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, K8 = K >> 3;
#pragma unroll
  for (int k = 0; k < PD_PW; ++k) {
    const int q = wv + PD_NW * k;
    if (2 * q < nr) {
      float a0[BM], a1[BM];
#pragma unroll
      for (int b = 0; b < BM; ++b) a0[b] = a1[b] = 0.f;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = lane + 64 * u;
        if (c < K8) {
#pragma unroll
          for (int b = 0; b < BM; ++b) {
            a0[b] = pd_dot8(wr[(2 * k) * U + u], gin[b * K8 + c], a0[b]);
            a1[b] = pd_dot8(wr[(2 * k + 1) * U + u], gin[b * K8 + c], a1[b]);
          }
        }
      }
      const int n = n0 + 2 * q;
#pragma unroll
      for (int b = 0; b < BM; ++b) {
        const float y0 = wave_sum(a0[b]), y1 = wave_sum(a1[b]);   // in every lane
        if (lane < rep)
          ll_store(dst + (size_t)lane * cst + (size_t)b * rw + (n >> 1),
                   pd_epi<E>(y0, y1, b, n, lam, xr, x0, d), tag);
      }
    }
  }
}

// Epilogue of this work-group's rows [n0, n0 + nr) and tagged stores of the
// bf16 pairs to dst (row stride rw words), to each of `rep` copies cst words
// apart.
template <int E, int BM>
__device__ __forceinline__ void pd_emit(float (*stage)[PD_RMAX], int n0, int nr, u64* dst, int rw,
                                        uint32_t tag, const float* lam, const bf16_t* xr,
                                        const bf16_t* x0, int d, int rep = 1, int cst = 0) {
  const int np = nr >> 1, tot = BM * np;
  for (int i = threadIdx.x; i < rep * tot; i += PD_T) {
    const int cp = i / tot, k = i - cp * tot;
    const int b = k / np, j = k - b * np, n = n0 + 2 * j;
    const uint32_t v = pd_epi<E>(stage[b][2 * j], stage[b][2 * j + 1], b, n, lam, xr, x0, d);
    ll_store(dst + (size_t)cp * cst + (size_t)b * rw + (n >> 1), v, tag);
  }
}

// DM, HM: the model dimension and head count as compile-time constants (0:
// read from P).  The kernel holds more uniform values than the 102 scalar
// registers of a wave and spills the rest to vector-register lanes, every
// reload an extra instruction in the phase that needs it; with d and H
// constant their derived sizes and the divisions by them fold away.  155M
// batch-1 generation (d 768, H 6): 171 -> 112 spilled scalars, 179.7 ->
// 168.0 ms (alternating A/B, three rounds, one box).  GR, the step's mode at
// compile time: 1 greedy without fp32 logits (no z, candidate or logits
// stores; 170.8 -> 169.6 ms on the same shape), 2 sampled without fp32 logits
// (z and candidates stored, no argmax keys); 0 reads it from P.
template <int DH, int BM, int UD, int DM = 0, int HM = 0, int GR = 0>
__global__ __launch_bounds__(PD_T) void k_decode_persist(PDParams P) {
  constexpr int KU = DH / 32;       // K slices per lane per chunk (4 lanes per key)
  constexpr int VD = DH / 64;       // output dims per lane in P.V
  constexpr int P2 = DH / 2, D4 = DH / 4;
  constexpr int PD_RING = DH == 128 ? 2 : 3;   // key chunks in flight per wave

  extern __shared__ uint4 lds4[];
  __shared__ float stage[BM][PD_RMAX];
  __shared__ float red[BM][PD_NW];
  __shared__ int s_pos[BM];
  __shared__ uint32_t s_in[3 * P2];   // raw q, k, v pairs of one head
  __shared__ uint32_t s_qp[P2];
  __shared__ uint32_t s_kp[P2];
  __shared__ float s_v[DH];
  __shared__ float s_o[PD_NW][DH];
  __shared__ float s_l[PD_NW];
  __shared__ u64 s_key[BM][PD_NW];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int G = gridDim.x, g = blockIdx.x;
  const int d = DM ? DM : P.d, H = HM ? HM : P.H, d2 = d >> 1;
  const bool greedy = GR ? GR == 1 : (P.greedy != 0);
  float* const logits = GR ? nullptr : P.logits;
  uint32_t* const cand = GR == 1 ? nullptr : P.cand;
  // exchange areas: with d and H constant, their offsets from xq and the
  // copy strides are compile-time constants (fewer live scalars)
  u64* const xq = P.xq;
  u64* const xp = DM ? xq + pd_layout(DM, HM ? HM : 1, 2) / 8 : P.xp;
  u64* const xm = DM ? xq + pd_layout(DM, HM ? HM : 1, 3) / 8 : P.xm;
  u64* const xh = DM ? xq + pd_layout(DM, HM ? HM : 1, 4) / 8 : P.xh;
  u64* const xx = DM ? xq + pd_layout(DM, HM ? HM : 1, 5) / 8 : P.xx;
  u64* const xk = DM ? xq + pd_layout(DM, HM ? HM : 1, 6) / 8 : P.xk;
  unsigned* const gen = DM ? (unsigned*)(xq + pd_layout(DM, HM ? HM : 1, 7) / 8) : P.gen;
  unsigned* const err = DM ? (unsigned*)(xq + pd_layout(DM, HM ? HM : 1, 8) / 8) : P.err;
  const int rep_stride = DM ? (int)pd_rep_stride(DM) : P.rep_stride;
  const int h_stride = DM ? (int)pd_h_stride(DM) : P.h_stride;
  const int p_stride = DM ? (int)pd_p_stride(DM, HM ? HM : 1) : P.p_stride;
  // this work-group's copy of the x' / x exchange (spreads the pollers of
  // each word over rep copies)
  const u64* xm_me = xm + (size_t)(g % P.rep) * rep_stride;
  const u64* xx_me = xx + (size_t)(g % P.rep) * rep_stride;
  bf16_t* sx0 = (bf16_t*)lds4;        // x0 (BM x d)
  bf16_t* sxs = sx0 + BM * d;         // layer input x
  bf16_t* sxm = sxs + BM * d;         // x after attention
  bf16_t* gin = sxm + BM * d;         // projection input (BM x d)
  bf16_t* ghb = gin + BM * d;         // proj input h (BM x 4d): its own buffer, since
                                      // waves poll it while others may still read gin
  float* spart = (float*)(ghb + BM * 4 * d);   // attention partials

  const uint32_t tb = __hip_atomic_load(gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) * PD_PH;
  if (tid < BM) s_pos[tid] = P.pos[tid];

  // layer 0's qkv weights first: their loads do not depend on the token
  uint4 wr[PD_SLOTS];
  {
    int n0, nr;
    pd_rows_qkv<P2>(P.head_xcd, H, d2, n0, nr);
    pd_wload2<UD>(P.layers + P.o_qkv, d, n0, nr, wr);
  }

  // ---- x = x0 = rms(embed[tok]) (every work-group, redundantly)
  for (int b = 0; b < BM; ++b) {
    int t = P.tok[b];
    t = t < 0 ? 0 : (t >= P.V ? P.V - 1 : t);
    const uint32_t* e = (const uint32_t*)(P.emb + (size_t)t * d);
    for (int i = tid; i < d2; i += PD_T) ((uint32_t*)gin)[b * d2 + i] = e[i];
  }
  __syncthreads();
  pd_rms<BM>(gin, sx0, d, P.eps, red);
  for (int i = tid; i < BM * d2; i += PD_T) ((uint32_t*)sxs)[i] = ((const uint32_t*)sx0)[i];
  __syncthreads();

  for (int l = 0; l < P.L; ++l) {
    const bf16_t* Wl = P.layers + P.lstride * l;
    const float* lam = P.lam + 8 * l;
    const bool lng = (P.long_mask >> l) & 1ull;
    const uint32_t t1 = tb + 5u * l + 1u;
    int n0, nr;

    // ---- 1: qkv
    pd_rows_qkv<P2>(P.head_xcd, H, d2, n0, nr);
    if (l > 0) pd_wload2<UD>(Wl + P.o_qkv, d, n0, nr, wr);
    if (l > 0) {
      ll_poll(xx_me, BM * d2, (uint32_t*)sxs, t1 - 1u, err);
      __syncthreads();
    }
    pd_rms<BM>(sxs, gin, d, P.eps, red);
    pd_wdot2<PE_STORE, UD, BM>(wr, (const uint4*)gin, d, n0, nr, xq, 3 * d2, t1, lam, nullptr,
                               nullptr, d, 1, 0);

    // ---- 2: attention of (b, h, split)
    const int S = lng ? P.s_long : P.s_win;
    const int NA = BM * H * S;   // attention units (b, h, s)
    const int au = pd_attn_unit(P.head_xcd, g, H, S, NA);
    const bool attn = au >= 0;
    // phase 3 (o projection) runs on up to P.on of the other work-groups,
    // whose weights load during the attention; the attention work-groups go
    // on to phase 4 (fewer producers of x' exchange faster: 8 rows each on
    // 96 work-groups measured 1.5% faster per step than 4-6 on 144-174)
    pd_rows_at(d2, n0, nr, attn ? -1 : pd_free_index(P.head_xcd, g, H, S, NA), min(P.on, G - NA));
    if (!attn) pd_wload2<UD>(Wl + P.o_o, d, n0, nr, wr);
    if (attn) {
      const int s = au % S, h = (au / S) % H, b = au / (S * H);
      const int p = s_pos[b];
      const int lo = lng ? 0 : max(0, p - P.window + 1);
      const int n = p - lo + 1;
      const int per = (n + S - 1) / S;
      const int k0 = lo + s * per;
      const int k1 = min(p + 1, k0 + per);
      const int nch = k1 > k0 ? (k1 - k0 + PD_KW - 1) / PD_KW : 0;
      // the wave index as a scalar: its chunk count and key positions are
      // uniform (scalar branches); part of the measured change above
      const int wvs = __builtin_amdgcn_readfirstlane(wv);
      const int nt = nch > wvs ? (nch - wvs + PD_NW - 1) / PD_NW : 0;
      const size_t ho = (((size_t)b * H + h) * P.max_ctx) * DH;
      bf16_t* kcl = P.kc + P.kvl * l;
      bf16_t* vcl = P.vc + P.kvl * l;
      const bf16_t* kh = kcl + ho;
      const bf16_t* vh = vcl + ho;
      const int sk = lane >> 2, sd = (lane & 3) * (DH / 4);   // score: key, first dim
      auto cbase = [&](int t) { return k0 + PD_KW * (wvs + PD_NW * t); };
      // K: 4 lanes x Dh/4 dims per key; V: every key's VD dims of this lane
      auto load = [&](int t, uint4* kr, uint32_t* vr) {
        const int c = cbase(t);
        const int j = c + sk;
        const bool ok = j < k1 && j != p;
#pragma unroll
        for (int u = 0; u < KU; ++u)
          kr[u] = ok ? *(const uint4*)(kh + (size_t)j * DH + sd + u * 8) : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int u = 0; u < PD_KW; ++u) {
          const int jj = c + u;
          const bool okv = jj < k1 && jj != p;
          if (VD == 2)
            vr[u] = okv ? *(const uint32_t*)(vh + (size_t)jj * DH + 2 * lane) : 0u;
          else
            vr[u] = okv ? (uint32_t)vh[(size_t)jj * DH + lane] : 0u;
        }
      };
      uint4 kb[PD_RING][KU];
      uint32_t vb[PD_RING][PD_KW];
#pragma unroll
      for (int r = 0; r < PD_RING - 1; ++r)
        if (r < nt) load(r, kb[r], vb[r]);
      // RoPE table entries of position p (independent of the wait below)
      float rc = 0.f, rsn = 0.f;
      if (tid < D4) {
        rc = P.cs[(size_t)p * D4 + tid];
        rsn = P.sn[(size_t)p * D4 + tid];
      }
      // q, k, v of this head from phase 1
      const u64* src = xq + (size_t)b * 3 * d2 + h * P2;
      for (int i = tid; i < 3 * P2; i += PD_T) {
        const int part = i / P2, k = i - part * P2;
        s_in[i] = ll_wait(src + part * d2 + k, t1, err);
      }
      __syncthreads();
      if (tid < 64) {   // QK-norm + RoPE, one dim pair per lane (lanes >= Dh/2 idle)
        const bool on = tid < P2;
        const uint32_t qw = on ? s_in[tid] : 0u, kw = on ? s_in[P2 + tid] : 0u;
        float q0 = __uint_as_float(qw << 16), q1 = __uint_as_float(qw & 0xffff0000u);
        float c0 = __uint_as_float(kw << 16), c1 = __uint_as_float(kw & 0xffff0000u);
        const float sq = wave_sum(q0 * q0 + q1 * q1);
        const float sk2 = wave_sum(c0 * c0 + c1 * c1);
        const float rq = rsqrtf(sq / (float)DH + P.eps), rk = rsqrtf(sk2 / (float)DH + P.eps);
        q0 = rbf(q0 * rq); q1 = rbf(q1 * rq);
        c0 = rbf(c0 * rk); c1 = rbf(c1 * rk);
        if (tid < D4) {
          const float c = rc, sn = rsn;
          const float a0 = c * q0 + sn * q1, a1 = c * q1 - sn * q0;
          const float b0 = c * c0 + sn * c1, b1 = c * c1 - sn * c0;
          q0 = a0; q1 = a1; c0 = b0; c1 = b1;
        }
        if (on) {
          const uint32_t vw = s_in[2 * P2 + tid];
          s_qp[tid] = pack2(q0, q1);
          const uint32_t kp = pack2(c0, c1);
          s_kp[tid] = kp;
          s_v[2 * tid] = __uint_as_float(vw << 16);
          s_v[2 * tid + 1] = __uint_as_float(vw & 0xffff0000u);
          if (k0 <= p && p < k1) {   // this split owns p: append to the cache
            const size_t ci = ho + (size_t)p * DH + 2 * tid;
            *(uint32_t*)(kcl + ci) = kp;
            *(uint32_t*)(vcl + ci) = vw;
          }
        }
      }
      __syncthreads();
      uint32_t qp[DH / 8];
#pragma unroll
      for (int e = 0; e < DH / 8; ++e) qp[e] = s_qp[sd / 2 + e];
      const float sl2 = P.scale * 1.4426950408889634f, sh2 = P.shift * 1.4426950408889634f;
      float acc[VD];
#pragma unroll
      for (int e = 0; e < VD; ++e) acc[e] = 0.f;
      float lsum = 0.f;   // wave-uniform
      auto compute = [&](int t, const uint4* kr, const uint32_t* vr) {
        const int c = cbase(t);
        const int j = c + sk;
        // a chunk without the new token (all but at most one per step) takes a
        // score and P.V path without the per-lane / per-key tests for it:
        // 165.8 -> 161.9 ms per 155M generation (two A/B steps)
        if (p < c || p >= c + PD_KW) {
          float sf = 0.f;
#pragma unroll
          for (int u = 0; u < KU; ++u) {
            sf = pd_dot2(qp[4 * u + 0], kr[u].x, sf);
            sf = pd_dot2(qp[4 * u + 1], kr[u].y, sf);
            sf = pd_dot2(qp[4 * u + 2], kr[u].z, sf);
            sf = pd_dot2(qp[4 * u + 3], kr[u].w, sf);
          }
          sf = quad_sum(sf);
          const float pf = j < k1 ? __builtin_amdgcn_exp2f(sf * sl2 - sh2) : 0.f;
#pragma unroll
          for (int u = 0; u < PD_KW; ++u) {
            const float pu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pf), 4 * u));
            lsum += pu;
            acc[0] += pu * __uint_as_float(vr[u] << 16);
            if (VD == 2) acc[VD - 1] += pu * __uint_as_float(vr[u] & 0xffff0000u);
          }
          return;
        }
        float sc = 0.f;
        if (j == p) {
#pragma unroll
          for (int e = 0; e < DH / 8; ++e) sc = pd_dot2(qp[e], s_kp[sd / 2 + e], sc);
        } else {
#pragma unroll
          for (int u = 0; u < KU; ++u) {
            sc = pd_dot2(qp[4 * u + 0], kr[u].x, sc);
            sc = pd_dot2(qp[4 * u + 1], kr[u].y, sc);
            sc = pd_dot2(qp[4 * u + 2], kr[u].z, sc);
            sc = pd_dot2(qp[4 * u + 3], kr[u].w, sc);
          }
        }
        sc = quad_sum(sc);
        const float pj = j < k1 ? __builtin_amdgcn_exp2f(sc * sl2 - sh2) : 0.f;
#pragma unroll
        for (int u = 0; u < PD_KW; ++u) {
          const float pu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pj), 4 * u));
          lsum += pu;
          float v0, v1 = 0.f;
          if (c + u == p) {
            v0 = s_v[VD * lane];
            if (VD == 2) v1 = s_v[VD * lane + 1];
          } else if (VD == 2) {
            v0 = __uint_as_float(vr[u] << 16);
            v1 = __uint_as_float(vr[u] & 0xffff0000u);
          } else {
            v0 = __uint_as_float(vr[u] << 16);
          }
          acc[0] += pu * v0;
          if (VD == 2) acc[VD - 1] += pu * v1;
        }
      };
      for (int t = 0; t < nt; t += PD_RING) {
#pragma unroll
        for (int r = 0; r < PD_RING; ++r) {
          if (t + r < nt) {
            const int tn = t + r + PD_RING - 1;
            if (tn < nt) load(tn, kb[(r + PD_RING - 1) % PD_RING], vb[(r + PD_RING - 1) % PD_RING]);
            compute(t + r, kb[r], vb[r]);
          }
        }
      }
#pragma unroll
      for (int e = 0; e < VD; ++e) s_o[wv][VD * lane + e] = acc[e];
      if (lane == 0) s_l[wv] = lsum;
      __syncthreads();
      u64* dst = xp + (size_t)au * (DH + 1);
      if (tid < DH) {
        float o = 0.f;
#pragma unroll
        for (int w = 0; w < PD_NW; ++w) o += s_o[w][tid];
        for (int c = 0; c < PD_REP_P; ++c)
          ll_store(dst + (size_t)c * p_stride + tid, __float_as_uint(o), t1 + 1u);
      }
      if (tid == 0) {
        float lt = 0.f;
#pragma unroll
        for (int w = 0; w < PD_NW; ++w) lt += s_l[w];
        for (int c = 0; c < PD_REP_P; ++c)
          ll_store(dst + (size_t)c * p_stride + DH, __float_as_uint(lt), t1 + 1u);
      }
    }

    // ---- 3: o = combine(partials); x' = mix_attn(x, x0, o Wo^T)
    // Every work-group without attention runs the poll and the combine, also
    // those that own no o rows (nr == 0): skipping them let those work-groups
    // start polling x' during the o projection, and the step measured 14%
    // slower (207.2 against 181.8 ms per 992-token generation, alternating
    // A/B on one box, identical tokens) -- pollers on the exchange lines slow
    // the exchange.
    if (!attn) {
      const int nw = BM * H * S * (DH + 1);
      ll_poll(xp + (size_t)(g % PD_REP_P) * p_stride, nw, (uint32_t*)spart, t1 + 1u, err);
      __syncthreads();
      for (int i = tid; i < BM * d; i += PD_T) {
        const int b = i / d, c = i - b * d, h = c / DH, e = c - h * DH;
        const float* pb = spart + (size_t)((b * H + h) * S) * (DH + 1);
        float o = 0.f, lt = 0.f;
        for (int s = 0; s < S; ++s) {
          o += pb[s * (DH + 1) + e];
          lt += pb[s * (DH + 1) + DH];
        }
        gin[i] = f2bf(o / lt);
      }
      __syncthreads();
      pd_wdot2<PE_ATTN, UD, BM>(wr, (const uint4*)gin, d, n0, nr, xm, d2, t1 + 2u, lam, sxs, sx0, d,
                                P.rep, rep_stride);
    }

    // ---- 4: h = relu2(rms(x') Wfc^T)
    pd_rows(2 * d, n0, nr, 0, G);
    pd_wload2<UD>(Wl + P.o_fc, d, n0, nr, wr);
    ll_poll(xm_me, BM * d2, (uint32_t*)sxm, t1 + 2u, err);
    __syncthreads();
    pd_rms<BM>(sxm, gin, d, P.eps, red);
    pd_wdot2<PE_RELU2, UD, BM>(wr, (const uint4*)gin, d, n0, nr, xh, 2 * d, t1 + 3u, lam, nullptr,
                               nullptr, d, PD_REP_H, h_stride);

    // ---- 5: x = mix_mlp(x', h Wproj^T)
    pd_rows(d2, n0, nr, 0, G);
    pd_wload<4 * UD, 1>(Wl + P.o_proj, 4 * d, n0, nr, wr);
    ll_poll(xh + (size_t)(g % PD_REP_H) * h_stride, BM * 2 * d, (uint32_t*)ghb, t1 + 3u, err);
    __syncthreads();
    pd_wdot<4 * UD, 1, BM>(wr, (const uint4*)ghb, 4 * d, nr, stage);
    pd_emit<PE_MLP, BM>(stage, n0, nr, xx, d2, t1 + 4u, lam, sxm, nullptr, d, P.rep, rep_stride);
  }

  // ---- lm_head over this work-group's rows [r0, r1), two register batches
  const uint32_t tl = tb + 5u * P.L;   // tag of the last x
  const int r0 = (int)((long long)P.V * g / G), r1 = (int)((long long)P.V * (g + 1) / G);
  // 18 16-byte chunks per lane and batch, two batches in flight: 0.3-0.6% per
  // step faster than 12; 24 (more registers for the whole kernel) slower
  constexpr int PD_HS = 18;
  constexpr int RB = PD_HS / UD;       // rows per wave per batch
  const int nrow = r1 - r0, nb = (nrow + PD_NW * RB - 1) / (PD_NW * RB);
  const int K8 = d >> 3;
  // Loads are unconditional (rows past this work-group's range and chunks
  // past the row read clamped addresses; hdot zeroes those chunks and drops
  // those rows), so the compiler can wait on one batch while the next is in
  // flight instead of on every load.
  auto hload = [&](int k, uint4* w) {
#pragma unroll
    for (int rr = 0; rr < RB; ++rr) {
      const int r = min(k * PD_NW * RB + wv + PD_NW * rr, nrow - 1);
      const uint4* row = (const uint4*)(P.head + (size_t)(r0 + r) * d);
#pragma unroll
      for (int u = 0; u < UD; ++u) w[rr * UD + u] = row[min(lane + 64 * u, K8 - 1)];
    }
  };
  u64 best[BM];
#pragma unroll
  for (int b = 0; b < BM; ++b) best[b] = 0ull;
  // sampled with candidates: this work-group's z (BM x nrow, nrow <= 4d and
  // <= 64 PD_ZE, host-checked) kept in the free h buffer
  bf16_t* zsl = ghb;
  auto hdot = [&](int k, const uint4* w) {
#pragma unroll
    for (int rr = 0; rr < RB; ++rr) {
      const int r = k * PD_NW * RB + wv + PD_NW * rr;
      if (r < nrow) {
        const int n = r0 + r;
        float acc[BM];
#pragma unroll
        for (int b = 0; b < BM; ++b) acc[b] = 0.f;
#pragma unroll
        for (int u = 0; u < UD; ++u) {
          // a chunk past the row adds exactly 0 (zero weights, finite x)
          const int c = lane + 64 * u;
          const bool cv = c < K8;
          const uint4 wz = cv ? w[rr * UD + u] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
          for (int b = 0; b < BM; ++b)
            acc[b] = pd_dot8(wz, ((const uint4*)gin)[b * K8 + (cv ? c : K8 - 1)], acc[b]);
        }
#pragma unroll
        for (int b = 0; b < BM; ++b) {
          const float y = wave_sum(acc[b]);
          const bf16_t zb = f2bf(y);
          if (greedy) {
            const u64 key = n < P.Vs ? (((u64)zkey(zb) << 16) | (u64)(0xffffu - (uint32_t)n)) : 0ull;
            best[b] = key > best[b] ? key : best[b];
          } else if (lane == 0) {
            P.z[(size_t)b * P.V + n] = zb;
            if (cand) zsl[b * nrow + r] = zb;
          }
          if (logits && lane == 0) logits[(size_t)b * P.V + n] = softcap(bf2f(zb));
        }
      }
    }
  };
  // batches in pairs (an odd count gets one batch of dropped rows); every
  // load unconditional, the last refill re-reads the last batch (unused)
  uint4 wa[PD_HS], wb[PD_HS];
  const int nbe = (nb + 1) & ~1;
  if (nb > 0) hload(0, wa);
  ll_poll(xx_me, BM * d2, (uint32_t*)sxs, tl, err);
  __syncthreads();
  pd_rms<BM>(sxs, gin, d, P.eps, red);
  for (int k = 0; k < nbe; k += 2) {
    hload(k + 1, wb);
    hdot(k, wa);
    hload(min(k + 2, nbe - 1), wa);
    hdot(k + 1, wb);
  }

  if (!greedy && cand) {
    // candidates of this work-group's slice (sample_cand): wave b < BM takes
    // row b, lane l the entries l + 64 i; TK_M + 1 rounds of a wave maximum
    // over the lanes' largest words, each popped from its lane
    __syncthreads();
    if (wv < BM) {
      const int b = wv;
      uint32_t w[PD_ZE];
#pragma unroll
      for (int i = 0; i < PD_ZE; ++i) {
        const int r = lane + 64 * i, n = r0 + r;
        w[i] = r < nrow && n < P.Vs
                   ? (zkey(zsl[b * nrow + r]) << 16) | (0xffffu - (uint32_t)n) : 0u;
      }
      uint32_t mine = 0u;   // lane e < TK_M: candidate e; lane TK_M: the next word
#pragma unroll 1
      for (int e = 0; e <= TK_M; ++e) {
        uint32_t lm = w[0];
#pragma unroll
        for (int i = 1; i < PD_ZE; ++i) lm = max(lm, w[i]);
        const uint32_t gm = __ockl_wfred_max_u32(lm);
        if (lane == e) mine = gm;
#pragma unroll
        for (int i = 0; i < PD_ZE; ++i) w[i] = w[i] == gm ? 0u : w[i];
      }
      if (lane < TK_M) cand[((size_t)b * G + g) * TK_M + lane] = mine;
      else if (lane == TK_M) P.cand_r[(size_t)b * G + g] = mine;
    }
  }
  if (greedy) {
    if (lane == 0) {
#pragma unroll
      for (int b = 0; b < BM; ++b) s_key[b][wv] = best[b];
    }
    __syncthreads();
    if (tid < BM) {
      u64 m = 0;
#pragma unroll
      for (int w = 0; w < PD_NW; ++w) m = s_key[tid][w] > m ? s_key[tid][w] : m;
      ll_store(xk + (size_t)g * BM + tid, (uint32_t)m, tl + 1u);
    }
    if (g == 0) {   // token = largest key over all work-groups
      u64 m[BM];
#pragma unroll
      for (int b = 0; b < BM; ++b) m[b] = 0ull;
      for (int i = tid; i < G; i += PD_T) {
#pragma unroll
        for (int b = 0; b < BM; ++b) {
          const u64 v = ll_wait(xk + (size_t)i * BM + b, tl + 1u, err);
          m[b] = v > m[b] ? v : m[b];
        }
      }
      __syncthreads();
#pragma unroll
      for (int b = 0; b < BM; ++b) {
        u64 v = m[b];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
          const u64 w = (u64)__shfl_xor((unsigned)v, o, 64);
          v = w > v ? w : v;
        }
        if (lane == 0) s_key[b][wv] = v;
      }
      __syncthreads();
      if (tid < BM) {
        u64 v = 0;
#pragma unroll
        for (int w = 0; w < PD_NW; ++w) v = s_key[tid][w] > v ? s_key[tid][w] : v;
        P.out_tok[tid] = (int32_t)(0xffffu - (uint32_t)(v & 0xffffu));
        P.pos[tid] = s_pos[tid] + 1;
      }
    }
  }
  // every work-group read the generation before its first output and work-
  // group 0 has consumed outputs of all of them: advance it for the next step
  if (g == 0 && tid == 0)
    __hip_atomic_store(gen, (tb / PD_PH) + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- host side --------------------------------------------------------------

int decode_persist_slots(int d) { return d <= 512 ? 1 : d <= 1024 ? 2 : d <= 1536 ? 3 : 0; }

// Row counts above one run for d <= 1024 (two 16-byte weight slots per lane):
// the row buffers and split partials of 2-4 rows at d 1536 leave the LDS
// budget too few splits.
bool decode_persist_fits(int B, int d, int H, int Dh, int V, int L, int G, int s_long) {
  const int ud = decode_persist_slots(d);
  if (B < 1 || B > PD_MAX_B || ud == 0 || (B > 1 && ud > 2) || (Dh != 64 && Dh != 128) ||
      d % 16 || V % 2 || V > 65536 || L > 50 || G < 1)
    return false;
  if (decode_persist_lds(B, d, H, Dh, s_long) > PD_MAX_LDS) return false;
  const int d2 = d / 2, rd = 2 * PD_PW * PD_NW;
  auto rows = [&](int npairs) { return 2 * ((npairs + G - 1) / G); };
  if (rows(3 * d2) > rd || rows(2 * d) > rd || rows(d2) > PD_NW) return false;
  // o projection over the work-groups without attention (fewest at the long layers)
  const int na = B * H * s_long;
  if (na >= G || s_long < 1 || 2 * ((d2 + (G - na) - 1) / (G - na)) > rd) return false;
  return true;
}

// Whether the step can keep each head's qkv rows and attention splits on XCD
// h: one row, G a multiple of 8 with the S attention splits of a head on
// work-groups h, h + 8, .., h + 8 (S - 1), at most 8 heads, and the head's
// 3 Dh/2 row pairs split into equal shares that each stay inside its q, k
// or v rows and fit a work-group's registers.
bool decode_persist_xcd_ok(int B, int d, int H, int Dh, int G, int s_long) {
  if (B != 1 || H < 1 || H > 8 || G < 8 || G % 8 || s_long < 1 || 8 * s_long > G ||
      H * Dh != d)
    return false;
  const int per = G / 8, p2 = Dh / 2;
  if ((3 * p2) % per) return false;
  const int q = 3 * p2 / per;
  return p2 % q == 0 && q <= PD_PW * PD_NW;
}

size_t decode_persist_lds(int B, int d, int H, int Dh, int s_long) {
  return (size_t)8 * B * d * 2 + (size_t)B * H * s_long * (Dh + 1) * 4;
}

// Launch of the G work-groups.  G is at most the CU count and a CU holds one
// (occupancy checked), so once the stream's earlier work has
// drained every work-group is resident; a plain launch is measured ~19 us per
// step cheaper than a cooperative one (which the runtime serialises), and the
// bounded waits end the kernel with the error flag set should residency ever
// fail.  coop: use the cooperative launch instead.
template <int DH, int BM, int UD, int DM = 0, int HM = 0, int GR = 0>
static hipError_t pd_launch(const PDParams& P, int G, size_t lds, bool coop, hipStream_t st) {
  const void* fn = (const void*)k_decode_persist<DH, BM, UD, DM, HM, GR>;
  static bool attr = false;
  if (!attr) {
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                             (int)PD_MAX_LDS);
    if (e != hipSuccess) return e;
    attr = true;
  }
  int nb = 0;
  hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, PD_T, lds);
  if (e != hipSuccess) return e;
  if (nb < 1) return hipErrorCooperativeLaunchTooLarge;
  PDParams a = P;
  void* args[] = {&a};
  if (coop) return hipLaunchCooperativeKernel(fn, dim3(G), dim3(PD_T), args, (unsigned)lds, st);
  return hipLaunchKernel(fn, dim3(G), dim3(PD_T), args, lds, st);
}

// Whether P's exchange areas and strides are the ones pd_layout places from
// P.xq (what a compile-time-shape instance assumes).
static bool pd_areas_match(const PDParams& P) {
  const size_t d = (size_t)P.d, H = (size_t)P.H;
  const char* q = (const char*)P.xq;
  const void* areas[7] = {P.xp, P.xm, P.xh, P.xx, P.xk, P.gen, P.err};
  for (int i = 0; i < 7; ++i)
    if ((const char*)areas[i] != q + pd_layout(d, H, i + 2)) return false;
  return (size_t)P.rep_stride == pd_rep_stride(d) && (size_t)P.h_stride == pd_h_stride(d) &&
         (size_t)P.p_stride == pd_p_stride(d, H);
}

template <int BM>
static hipError_t pd_dispatch(const PDParams& P, int Dh, int G, size_t lds, bool coop,
                              bool spec, hipStream_t st) {
  // the 155M model's shape (d 768, H 6 x 128) at 1-4 rows: its own instances
  // (which derive the exchange areas from xq: the caller's must match), the
  // mode constant where no fp32 logits are asked for; 2 / 3 rows 245 -> 224 /
  // 294 -> 267 us per step (positions 520-647)
  if (spec && Dh == 128 && P.d == 768 && P.H == 6) {
    if (!pd_areas_match(P)) return hipErrorInvalidValue;
    if (!P.logits)
      return P.greedy ? pd_launch<128, BM, 2, 768, 6, 1>(P, G, lds, coop, st)
                      : pd_launch<128, BM, 2, 768, 6, 2>(P, G, lds, coop, st);
    return pd_launch<128, BM, 2, 768, 6>(P, G, lds, coop, st);
  }
  switch (Dh * 16 + decode_persist_slots(P.d)) {
    case 64 * 16 + 1: return pd_launch<64, BM, 1>(P, G, lds, coop, st);
    case 64 * 16 + 2: return pd_launch<64, BM, 2>(P, G, lds, coop, st);
    case 128 * 16 + 1: return pd_launch<128, BM, 1>(P, G, lds, coop, st);
    case 128 * 16 + 2: return pd_launch<128, BM, 2>(P, G, lds, coop, st);
    default: break;
  }
  if constexpr (BM == 1) {   // three weight slots (d up to 1536): one row only
    switch (Dh * 16 + decode_persist_slots(P.d)) {
      case 64 * 16 + 3: return pd_launch<64, 1, 3>(P, G, lds, coop, st);
      case 128 * 16 + 3: return pd_launch<128, 1, 3>(P, G, lds, coop, st);
      default: break;
    }
  }
  return hipErrorInvalidValue;
}

hipError_t decode_persist(const PDParams& P, int B, int Dh, int G, bool coop, bool specialize,
                          hipStream_t st) {
  const size_t lds = decode_persist_lds(B, P.d, P.H, Dh, P.s_long);
  if (lds > PD_MAX_LDS || B < 1 || B > PD_MAX_B) return hipErrorInvalidValue;
  // the attention work-groups leave at least one for the o rows, each within
  // what its registers hold
  const int rd = 2 * PD_PW * PD_NW;
  const int no = P.on < G - B * P.H * P.s_long ? P.on : G - B * P.H * P.s_long;
  if (no < 1 || 2 * ((P.d / 2 + no - 1) / no) > rd) return hipErrorInvalidValue;
  if (P.head_xcd && !decode_persist_xcd_ok(B, P.d, P.H, Dh, G, P.s_long))
    return hipErrorInvalidValue;
  switch (B) {
    case 1: return pd_dispatch<1>(P, Dh, G, lds, coop, specialize, st);
    case 2: return pd_dispatch<2>(P, Dh, G, lds, coop, specialize, st);
    case 3: return pd_dispatch<3>(P, Dh, G, lds, coop, specialize, st);
    case 4: return pd_dispatch<4>(P, Dh, G, lds, coop, specialize, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ann
