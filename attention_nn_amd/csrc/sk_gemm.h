// Skinny MFMA GEMM body (decode projections, M <= 128): one 16T x 16T
// output tile of C = A W^T per work-group (tile column bx, row by); the four
// waves split K into quarters and each loads its whole quarter of A and W
// fragments (up to SK_KB k-steps of 32) into registers before the first MFMA,
// so a launch waits on memory about once.  The partial tiles are summed
// through LDS in wave order (deterministic).  RMS: the rows of A are
// normalised in the kernel -- per-wave sums of squares over the quarter,
// exchanged through LDS, scale = rsqrt(mean + eps), x * scale rounded to bf16
// before the MFMA (model.py:48-49 with the bf16 output of an eager op); needs
// K <= 3072.  Wave 0 hands each 4-row group to store(m, n, v): column n of
// rows m .. m + 3 (fp32 sums; rows past M and columns past N are the caller's
// to drop).
#pragma once
#include "common.h"

namespace ann {

typedef __bf16 sk_bf16x8_t __attribute__((ext_vector_type(8)));
typedef float sk_floatx4_t __attribute__((ext_vector_type(4)));

constexpr int SK_KB = 24;   // largest batch of k-steps per wave

template <bool RMS, int KB, int T, typename Store>
__device__ __forceinline__ void gemm_sk_body(const bf16_t* __restrict__ A, int lda,
                                             const bf16_t* __restrict__ W, int M, int N, int K,
                                             float eps, int bx, int by, Store&& store) {
  // work-group tile (16 T) x (16 T): T x T blocks of 16x16 per wave
  __shared__ sk_floatx4_t red[3][T * T][64];
  __shared__ float s_ss[4][16 * T];
  const int tid = threadIdx.x, lane = tid & 63, wk = tid >> 6;
  const int n0 = bx * 16 * T, m0 = by * 16 * T;
  const int kw = K >> 7;   // k-steps per wave
  const int r16 = lane & 15, kq = (lane >> 4) * 8;
  const bf16_t* ap[T];
  const bf16_t* wp[T];
  bool aok[T], wok[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int arow = m0 + 16 * t + r16, wrow = n0 + 16 * t + r16;
    aok[t] = arow < M;
    wok[t] = wrow < N;
    ap[t] = A + (size_t)(aok[t] ? arow : 0) * lda + wk * kw * 32 + kq;
    wp[t] = W + (size_t)(wok[t] ? wrow : 0) * K + wk * kw * 32 + kq;
  }
  sk_floatx4_t acc[T][T];
#pragma unroll
  for (int i = 0; i < T; ++i)
#pragma unroll
    for (int j = 0; j < T; ++j) acc[i][j] = sk_floatx4_t{0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < kw; s0 += KB) {
    uint4 ca[KB][T], cw[KB][T];
    // every load unconditional (rows clamped in ap / wp, k-steps past the
    // wave's range re-read its last one), so they issue back to back with
    // no branch: a row past M or N only feeds outputs that are never stored,
    // and k-steps past the range are zeroed once all loads are in flight
#pragma unroll
    for (int i = 0; i < KB; ++i) {
      const int ks = min(s0 + i, kw - 1);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        ca[i][t] = *(const uint4*)(ap[t] + ks * 32);
        cw[i][t] = *(const uint4*)(wp[t] + ks * 32);
      }
    }
#pragma unroll
    for (int i = 0; i < KB; ++i)
      if (s0 + i >= kw) {
#pragma unroll
        for (int t = 0; t < T; ++t) ca[i][t] = cw[i][t] = make_uint4(0, 0, 0, 0);
      }
    float scale[T];
#pragma unroll
    for (int t = 0; t < T; ++t) scale[t] = 1.f;
    if (RMS) {   // the host guarantees kw <= KB: one pass, uniform barrier
#pragma unroll
      for (int t = 0; t < T; ++t) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < KB; ++i) {
          float f[8];
          unpack8(ca[i][t], f);
#pragma unroll
          for (int j = 0; j < 8; ++j) ss += f[j] * f[j];
        }
        ss += __shfl_xor(ss, 16, 64);
        ss += __shfl_xor(ss, 32, 64);
        if (lane < 16) s_ss[wk][16 * t + lane] = ss;
      }
      __syncthreads();
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int r = 16 * t + r16;
        const float tt = ((s_ss[0][r] + s_ss[1][r]) + s_ss[2][r]) + s_ss[3][r];
        scale[t] = rsqrtf(tt / (float)K + eps);
      }
    }
#pragma unroll
    for (int i = 0; i < KB; ++i) {
      if (s0 + i < kw) {
        uint4 a[T];
#pragma unroll
        for (int t = 0; t < T; ++t) {
          a[t] = ca[i][t];
          if (RMS) {
            float f[8];
            unpack8(a[t], f);
            a[t].x = pack2(f[0] * scale[t], f[1] * scale[t]);
            a[t].y = pack2(f[2] * scale[t], f[3] * scale[t]);
            a[t].z = pack2(f[4] * scale[t], f[5] * scale[t]);
            a[t].w = pack2(f[6] * scale[t], f[7] * scale[t]);
          }
        }
#pragma unroll
        for (int ta = 0; ta < T; ++ta)
#pragma unroll
          for (int tw = 0; tw < T; ++tw)
            acc[ta][tw] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                *(sk_bf16x8_t*)&a[ta], *(sk_bf16x8_t*)&cw[i][tw], acc[ta][tw], 0, 0, 0);
      }
    }
  }
  if (wk > 0) {
#pragma unroll
    for (int ta = 0; ta < T; ++ta)
#pragma unroll
      for (int tw = 0; tw < T; ++tw) red[wk - 1][ta * T + tw][lane] = acc[ta][tw];
  }
  __syncthreads();
  if (wk > 0) return;
#pragma unroll
  for (int ta = 0; ta < T; ++ta)
#pragma unroll
    for (int tw = 0; tw < T; ++tw) {
      sk_floatx4_t v = acc[ta][tw];
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const sk_floatx4_t p = red[j][ta * T + tw][lane];
        v[0] += p[0];
        v[1] += p[1];
        v[2] += p[2];
        v[3] += p[3];
      }
      // lane: column n0 + 16 tw + r16 of rows m0 + 16 ta + 4 (lane >> 4) + r;
      // every lane of wave 0 calls store (a store may exchange across lanes)
      store(m0 + 16 * ta + (lane >> 4) * 4, n0 + 16 * tw + r16, v);
    }
}


}  // namespace ann
