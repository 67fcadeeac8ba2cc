// Epilogues shared by the MFMA GEMM kernels (device code, internal).
#pragma once
#include "common.h"
#include "launch.h"

namespace ann {

// QKV epilogue of one BM x 128 tile whose bf16 values are staged in LDS
// (row pitch PITCH bf16, a multiple of 8): two threads per row take 64
// columns each, 256 threads, so a thread has QKV_ROWS(BM) rows.  A tile lies
// in one section (q, k or v) and holds one head (Dh 128) or two (Dh 64).  q
// and k: fp32 sum of squares over the head, x * rsqrt(mean + eps) rounded to
// bf16, then the dim pairs below Dh/4 rotated by the RoPE table row of the
// token's position (model.py:244-247); v is copied.  16-byte stores.
//
// The token positions and this thread's 16 cos / sin pairs of each row come
// from qkv_prefetch, issued before the tile is staged: loaded inside the row
// loop they were two dependent global round trips per row.
template <int BM>
struct QkvRows {
  static constexpr int R = (BM + 127) / 128;
  int ps[R];
  float4 c[R][4], s[R][4];
};

template <int BM>
__device__ __forceinline__ void qkv_prefetch(const EpiArgs& ea, int m0, int M, int tid,
                                             QkvRows<BM>& pr) {
  const int Dh = ea.Dh, D4 = Dh / 4;
  const int d0 = Dh == 128 ? 32 * (tid & 1) : 0;
#pragma unroll
  for (int k = 0; k < QkvRows<BM>::R; ++k) {
    const int m = min(m0 + (tid >> 1) + 128 * k, M - 1);
    const int b = m / ea.T;
    pr.ps[k] = ea.pos[b] + (m - b * ea.T);
  }
#pragma unroll
  for (int k = 0; k < QkvRows<BM>::R; ++k) {
    const float4* cp = (const float4*)(ea.cs + (size_t)pr.ps[k] * D4 + d0 / 2);
    const float4* sp = (const float4*)(ea.sn + (size_t)pr.ps[k] * D4 + d0 / 2);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      pr.c[k][g] = cp[g];
      pr.s[k][g] = sp[g];
    }
  }
}

template <int BM, int PITCH>
__device__ __forceinline__ void qkv_tile_epilogue(const EpiArgs& ea, const bf16_t* tile, int m0,
                                                  int n0, int M, int tid, const QkvRows<BM>& pr) {
  static_assert(PITCH % 8 == 0, "16-byte rows");
  constexpr int CP = PITCH;
  const int Dh = ea.Dh, d = ea.H * Dh;
  const int sec = n0 / d;                   // 0 q, 1 k, 2 v
  const int half = tid & 1;
  const int head = (n0 - sec * d) / Dh + (Dh == 64 ? half : 0);
  // this thread's two 32-dim runs inside its head: the rotated pairs (dims
  // below Dh/2) are the first run, split evenly between the two threads of a
  // row for Dh 128 (dims 32h.. and 64 + 32h..), the head's halves for Dh 64
  const int d0 = Dh == 128 ? 32 * half : 0;
  const int d1 = Dh == 128 ? 64 + 32 * half : 32;
  const int c0 = Dh == 128 ? 32 * half : 64 * half;   // tile columns of the runs
  const int c1 = c0 + (Dh == 128 ? 64 : 32);
#pragma unroll
  for (int k = 0; k < QkvRows<BM>::R; ++k) {
    const int rr = (tid >> 1) + 128 * k;
    const int m = m0 + rr;
    if (rr >= BM || m >= M) continue;       // both threads of a pair skip together
    uint4 v[8];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      v[u] = *(const uint4*)(tile + rr * CP + c0 + u * 8);
      v[4 + u] = *(const uint4*)(tile + rr * CP + c1 + u * 8);
    }
    const int b = m / ea.T;
    const int ps = pr.ps[k];
    if (sec < 2) {
      float f[64];
#pragma unroll
      for (int u = 0; u < 8; ++u) unpack8(v[u], f + 8 * u);
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 64; ++e) ss += f[e] * f[e];
      if (Dh == 128) ss += __shfl_xor(ss, 1, 64);
      const float r = rsqrtf(ss / (float)Dh + ea.eps);
      // rounded to bf16 a pair at a time
#pragma unroll
      for (int e = 0; e < 64; e += 2) {
        const uint32_t w = pack2(f[e] * r, f[e + 1] * r);
        f[e] = lo_f(w);
        f[e + 1] = hi_f(w);
      }
      // pairs d0/2 .. d0/2 + 15 are all below Dh/4: rotate them
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 c4 = pr.c[k][g], s4 = pr.s[k][g];
        const float cc[4] = {c4.x, c4.y, c4.z, c4.w}, ssn[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int jp = 4 * g + e;
          const float a0 = f[2 * jp], a1 = f[2 * jp + 1];
          f[2 * jp] = cc[e] * a0 + ssn[e] * a1;
          f[2 * jp + 1] = cc[e] * a1 - ssn[e] * a0;
        }
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
        v[u] = make_uint4(pack2(f[8 * u], f[8 * u + 1]), pack2(f[8 * u + 2], f[8 * u + 3]),
                          pack2(f[8 * u + 4], f[8 * u + 5]), pack2(f[8 * u + 6], f[8 * u + 7]));
    }
    bf16_t* hb = sec == 0 ? ea.out + (size_t)m * ea.ldo + head * Dh
                          : (sec == 1 ? ea.kc : ea.vc) +
                                (((size_t)b * ea.H + head) * ea.max_ctx + ps) * Dh;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      *(uint4*)(hb + d0 + u * 8) = v[u];
      *(uint4*)(hb + d1 + u * 8) = v[4 + u];
    }
  }
}

}  // namespace ann
