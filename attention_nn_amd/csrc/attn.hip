// Causal / sliding-window attention of query rows against the bf16 KV cache
// (model.py:248-254): keep key j for query position p iff j <= p and, on the
// windowed layers, p - j < window.  Scores 0.1 * q.k in fp32, online softmax in
// fp32, P.V accumulated in fp32, output rounded once to bf16.
//
// Grid (nsplit, H, M): one work-group per (query row, head, key split).  A
// windowed layer touches only its last `window` keys; a full layer all p + 1.
// Keys are visited in chunks of 64: 16 lanes x 16 B read one 256-B key row
// (Dh = 128), P.V lanes own one dim pair and read 256-B V rows, softmax
// statistics are wave-shuffle reductions.  nsplit > 1 (decode, few rows)
// writes unnormalised partials (o, m, l) merged by k_attn_combine.
#include <math.h>
#include "common.h"
#include "launch.h"

namespace ann {

constexpr int ATT_KC = 64;       // keys per chunk
constexpr int ATT_THREADS = 256;

template <int DH>
__global__ __launch_bounds__(ATT_THREADS) void k_attn(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ kc, const bf16_t* __restrict__ vc,
    const int32_t* __restrict__ pos, bf16_t* __restrict__ out, float* __restrict__ part, int T,
    int H, int max_ctx, int window, int is_long, float scale, int nsplit) {
  constexpr int LPK = DH / 8;              // lanes per key (16-byte slices)
  constexpr int KPW = 64 / LPK;            // keys per wave per pass
  constexpr int KW = ATT_KC / 4;           // keys per wave per chunk
  constexpr int NPAIR = DH / 2;            // P.V lanes per key
  constexpr int NSUB = ATT_THREADS / NPAIR;  // key subsets in P.V

  __shared__ float s_sc[ATT_KC];
  __shared__ float s_p[ATT_KC];
  __shared__ float s_stat[2];
  __shared__ float s_o[NSUB][DH];

  const int split = blockIdx.x, h = blockIdx.y, m = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int b = m / T, t = m % T;
  const int d = H * DH;
  const int p = pos[b] + t;
  const int lo = is_long ? 0 : max(0, p - window + 1);
  const int n = p - lo + 1;
  const int nchunks = (n + ATT_KC - 1) / ATT_KC;
  const int cps = (nchunks + nsplit - 1) / nsplit;
  const int c_begin = split * cps;
  const int c_end = min(nchunks, c_begin + cps);

  const size_t head_off = ((size_t)b * H + h) * max_ctx;
  const bf16_t* kh = kc + head_off * DH;
  const bf16_t* vh = vc + head_off * DH;

  const int kl = lane / LPK, dl = lane % LPK;
  float qf[8];
  unpack8(*(const uint4*)(q + (size_t)m * d + h * DH + dl * 8), qf);

  const int dp = tid % NPAIR, ks = tid / NPAIR;
  float o0 = 0.f, o1 = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  for (int c = c_begin; c < c_end; ++c) {
    const int kb = lo + c * ATT_KC;
    const int kn = min(ATT_KC, p + 1 - kb);
#pragma unroll
    for (int ps = 0; ps < KW / KPW; ++ps) {
      const int j = wv * KW + ps * KPW + kl;
      float s = 0.f;
      if (j < kn) {
        float kf[8];
        unpack8(*(const uint4*)(kh + (size_t)(kb + j) * DH + dl * 8), kf);
#pragma unroll
        for (int e = 0; e < 8; ++e) s += qf[e] * kf[e];
      }
      s = group_sum<LPK>(s);
      if (dl == 0) s_sc[j] = j < kn ? s * scale : -INFINITY;
    }
    __syncthreads();
    if (wv == 0) {
      const float s = s_sc[lane];
      const float mc = group_max<64>(s);
      const float mn = fmaxf(m_run, mc);
      const float e = expf(s - mn);
      s_p[lane] = e;
      const float ls = group_sum<64>(e);
      if (lane == 0) {
        s_stat[0] = mn;
        s_stat[1] = ls;
      }
    }
    __syncthreads();
    const float mn = s_stat[0];
    const float f = expf(m_run - mn);   // 0 on the first chunk (m_run = -inf)
    l_run = l_run * f + s_stat[1];
    o0 *= f;
    o1 *= f;
    m_run = mn;
    for (int j = ks; j < kn; j += NSUB) {
      const float pj = s_p[j];
      const uint32_t vw = *(const uint32_t*)(vh + (size_t)(kb + j) * DH + 2 * dp);
      o0 += pj * __uint_as_float(vw << 16);
      o1 += pj * __uint_as_float(vw & 0xffff0000u);
    }
    __syncthreads();
  }
  s_o[ks][2 * dp] = o0;
  s_o[ks][2 * dp + 1] = o1;
  __syncthreads();
  if (tid < DH) {
    float o = 0.f;
#pragma unroll
    for (int i = 0; i < NSUB; ++i) o += s_o[i][tid];
    if (nsplit == 1) {
      out[(size_t)m * d + h * DH + tid] = f2bf(o / l_run);
    } else {
      float* pp = part + (((size_t)m * H + h) * nsplit + split) * (DH + 2);
      pp[tid] = o;
      if (tid == 0) {
        pp[DH] = m_run;
        pp[DH + 1] = l_run;
      }
    }
  }
}

// Merge the nsplit partials of one (row, head): o = sum_s e^(m_s - M) o_s / L.
template <int DH>
__global__ void k_attn_combine(const float* __restrict__ part, bf16_t* __restrict__ out, int H,
                               int nsplit) {
  const int h = blockIdx.x, m = blockIdx.y, tid = threadIdx.x;
  const float* pp = part + ((size_t)m * H + h) * nsplit * (DH + 2);
  float M = -INFINITY;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, pp[s * (DH + 2) + DH]);
  float L = 0.f, o = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    const float ms = pp[s * (DH + 2) + DH];
    if (ms == -INFINITY) continue;
    const float f = expf(ms - M);
    L += f * pp[s * (DH + 2) + DH + 1];
    o += f * pp[s * (DH + 2) + tid];
  }
  out[(size_t)m * H * DH + h * DH + tid] = f2bf(o / L);
}

hipError_t attention(const bf16_t* q, const bf16_t* kc, const bf16_t* vc, const int32_t* pos,
                     bf16_t* out, float* part, int M, int T, int H, int Dh, int max_ctx,
                     int window, bool long_layer, float scale, int nsplit, hipStream_t st) {
  if (nsplit < 1 || M <= 0) return hipErrorInvalidValue;
  dim3 grid(nsplit, H, M);
  switch (Dh) {
#define ANN_ATT_CASE(D)                                                                        \
  case D:                                                                                      \
    hipLaunchKernelGGL(k_attn<D>, grid, dim3(ATT_THREADS), 0, st, q, kc, vc, pos, out, part, T, \
                       H, max_ctx, window, (int)long_layer, scale, nsplit);                   \
    if (nsplit > 1)                                                                            \
      hipLaunchKernelGGL(k_attn_combine<D>, dim3(H, M), dim3(D), 0, st, part, out, H, nsplit); \
    break;
    ANN_ATT_CASE(64)
    ANN_ATT_CASE(128)
#undef ANN_ATT_CASE
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace ann
