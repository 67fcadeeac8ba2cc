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
// o = sum_s O_s / sum_s L_s (rounded once to bf16) is formed by the last split
// of (b, h) to finish: partials go out with coherent (sc1) stores, a device
// counter per (b, h) elects that split, which reads them back in split order
// (deterministic) and resets the counter.
//
// Chunk of 64 keys: 4 lanes x 64 B read one 256-B key row (Dh = 128); for
// P.V 16 lanes x 16 B cover a V row, 16 key groups accumulate in registers
// and are reduced once through LDS at the end.
#include <math.h>
#include "common.h"
#include "launch.h"

namespace ann {

constexpr int AD_KC = 64;
constexpr int AD_THREADS = 256;

template <int DH>
__global__ __launch_bounds__(AD_THREADS) void k_attn_dec(
    const bf16_t* __restrict__ qkv, bf16_t* __restrict__ kc, bf16_t* __restrict__ vc,
    const int32_t* __restrict__ pos, const float* __restrict__ cs, const float* __restrict__ sn,
    float* __restrict__ part, unsigned* __restrict__ cnt, bf16_t* __restrict__ out, int H,
    int max_ctx, int window, int is_long, float scale, float shift, float eps, int nsplit) {
  constexpr int TPK = AD_THREADS / AD_KC;   // threads per key in the score pass (4)
  constexpr int DPT = DH / TPK;             // dims per thread in the score pass
  constexpr int VL = DH / 8;                // lanes per V row (16-byte slices)
  constexpr int NG = AD_THREADS / VL;       // key groups in the P.V pass
  constexpr int P = DH / 2, D4 = DH / 4;

  __shared__ float s_q[DH];
  __shared__ float s_k[DH];
  __shared__ float s_v[DH];
  __shared__ float s_p[AD_KC];
  __shared__ float s_o[NG][DH + 1];
  __shared__ float s_l[AD_THREADS / 64];

  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int d = H * DH;
  const int p = pos[b];
  const int lo = is_long ? 0 : max(0, p - window + 1);
  const int n = p - lo + 1;
  const int per = (n + nsplit - 1) / nsplit;
  const int k0 = lo + split * per;
  const int k1 = min(p + 1, k0 + per);

  const size_t head_off = ((size_t)b * H + h) * max_ctx;
  const bf16_t* kh = kc + head_off * DH;
  const bf16_t* vh = vc + head_off * DH;
  const int kk = tid / TPK, qd = (tid % TPK) * DPT;
  const int vd = (tid % VL) * 8, vg = tid / VL;
  constexpr int KU = DPT / 8;          // 16-byte K slices per thread per chunk
  constexpr int VU = AD_KC / NG;       // V rows per thread per chunk

  // K/V of a chunk straight into registers (the key at p comes from LDS)
  auto load_chunk = [&](int c, uint4* kr, uint4* vr) {
    const int j = c + kk;
    const bool ok = j < k1 && j != p;
#pragma unroll
    for (int u = 0; u < KU; ++u)
      kr[u] = ok ? *(const uint4*)(kh + (size_t)j * DH + qd + u * 8) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < VU; ++u) {
      const int jj = c + vg + u * NG;
      vr[u] = (jj < k1 && jj != p) ? *(const uint4*)(vh + (size_t)jj * DH + vd)
                                   : make_uint4(0, 0, 0, 0);
    }
  };
  uint4 ka[KU], va[VU];
  if (k0 < k1) load_chunk(k0, ka, va);   // independent of q: overlaps the prologue

  // ---- new token: QK-norm + RoPE (one dim pair per lane)
  if (tid < P) {
    const bf16_t* row = qkv + (size_t)b * 3 * d + h * DH + 2 * tid;
    const uint32_t qw = *(const uint32_t*)row;
    const uint32_t kw = *(const uint32_t*)(row + d);
    const uint32_t vw = *(const uint32_t*)(row + 2 * d);
    float q0 = __uint_as_float(qw << 16), q1 = __uint_as_float(qw & 0xffff0000u);
    float c0 = __uint_as_float(kw << 16), c1 = __uint_as_float(kw & 0xffff0000u);
    const float sq = group_sum<P>(q0 * q0 + q1 * q1);
    const float sk = group_sum<P>(c0 * c0 + c1 * c1);
    const float rq = rsqrtf(sq / (float)DH + eps), rk = rsqrtf(sk / (float)DH + eps);
    q0 = rbf(q0 * rq); q1 = rbf(q1 * rq);
    c0 = rbf(c0 * rk); c1 = rbf(c1 * rk);
    if (tid < D4) {
      const float c = cs[(size_t)p * D4 + tid], s = sn[(size_t)p * D4 + tid];
      const float a0 = c * q0 + s * q1, a1 = c * q1 - s * q0;
      const float b0 = c * c0 + s * c1, b1 = c * c1 - s * c0;
      q0 = a0; q1 = a1; c0 = b0; c1 = b1;
    }
    q0 = rbf(q0); q1 = rbf(q1); c0 = rbf(c0); c1 = rbf(c1);
    s_q[2 * tid] = q0; s_q[2 * tid + 1] = q1;
    s_k[2 * tid] = c0; s_k[2 * tid + 1] = c1;
    s_v[2 * tid] = __uint_as_float(vw << 16);
    s_v[2 * tid + 1] = __uint_as_float(vw & 0xffff0000u);
    if (k0 <= p && p < k1) {   // this work-group owns position p: append to the cache
      const size_t ci = (((size_t)b * H + h) * max_ctx + p) * DH + 2 * tid;
      *(uint32_t*)(kc + ci) = pack2(c0, c1);
      *(uint32_t*)(vc + ci) = vw;
    }
  }
  __syncthreads();

  float qf[DPT];
#pragma unroll
  for (int e = 0; e < DPT; ++e) qf[e] = s_q[qd + e];
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  float lsum = 0.f;

  for (int c = k0; c < k1; c += AD_KC) {
    uint4 kb[KU], vb[VU];
    const bool more = c + AD_KC < k1;
    if (more) load_chunk(c + AD_KC, kb, vb);   // next chunk in flight during this one
    const int kn = min(AD_KC, k1 - c);
    {
      const int j = c + kk;
      float s = 0.f;
      if (kk < kn) {
        if (j == p) {
#pragma unroll
          for (int e = 0; e < DPT; ++e) s += qf[e] * s_k[qd + e];
        } else {
#pragma unroll
          for (int u = 0; u < KU; ++u) {
            float kf[8];
            unpack8(ka[u], kf);
#pragma unroll
            for (int e = 0; e < 8; ++e) s += qf[u * 8 + e] * kf[e];
          }
        }
      }
      s = group_sum<TPK>(s);
      if (tid % TPK == 0) s_p[kk] = kk < kn ? expf(s * scale - shift) : 0.f;
    }
    __syncthreads();
    if (tid < AD_KC) lsum += s_p[tid];
#pragma unroll
    for (int u = 0; u < VU; ++u) {
      const int kv = vg + u * NG;
      if (kv < kn) {
        const float pj = s_p[kv];
        float vf[8];
        if (c + kv == p) {
#pragma unroll
          for (int e = 0; e < 8; ++e) vf[e] = s_v[vd + e];
        } else {
          unpack8(va[u], vf);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += pj * vf[e];
      }
    }
    __syncthreads();
    if (more) {
#pragma unroll
      for (int u = 0; u < KU; ++u) ka[u] = kb[u];
#pragma unroll
      for (int u = 0; u < VU; ++u) va[u] = vb[u];
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) s_o[vg][vd + e] = acc[e];
  lsum = group_sum<64>(lsum);
  if ((tid & 63) == 0) s_l[tid >> 6] = lsum;
  __syncthreads();
  // partial (O, L) of this split with coherent stores; the last split of
  // (b, h) to arrive sums all of them in split order and writes o = O / L
  float* pbase = part + ((size_t)b * H + h) * nsplit * (DH + 1);
  float* pp = pbase + (size_t)split * (DH + 1);
  if (tid < DH) {
    float o = 0.f;
#pragma unroll
    for (int g = 0; g < NG; ++g) o += s_o[g][tid];
    __hip_atomic_store(pp + tid, o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (tid == 0) {
    float l = 0.f;
    for (int w = 0; w < AD_THREADS / 64; ++w) l += s_l[w];
    __hip_atomic_store(pp + DH, l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (nsplit == 1) {
    __syncthreads();
    if (tid < DH) {
      const float o = __hip_atomic_load(pp + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const float l = __hip_atomic_load(pp + DH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      out[(size_t)b * d + h * DH + tid] = f2bf(o / l);
    }
    return;
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  __shared__ unsigned s_last;
  if (tid == 0) {
    const unsigned old = __hip_atomic_fetch_add(cnt + b * H + h, 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    s_last = old == (unsigned)nsplit - 1;
  }
  __syncthreads();
  if (!s_last) return;
  if (tid < DH) {
    float o = 0.f, l = 0.f;
    for (int sp = 0; sp < nsplit; ++sp) {
      o += __hip_atomic_load(pbase + (size_t)sp * (DH + 1) + tid, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      l += __hip_atomic_load(pbase + (size_t)sp * (DH + 1) + DH, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    }
    out[(size_t)b * d + h * DH + tid] = f2bf(o / l);
  }
  if (tid == 0) __hip_atomic_store(cnt + b * H + h, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

hipError_t attn_decode(const bf16_t* qkv, bf16_t* kc, bf16_t* vc, const int32_t* pos,
                       const float* cs, const float* sn, float* part, unsigned* cnt, bf16_t* out,
                       int B, int H, int Dh, int max_ctx, int window, bool long_layer, float scale,
                       float eps, int nsplit, hipStream_t st) {
  if (nsplit < 1 || B <= 0) return hipErrorInvalidValue;
  const float shift = scale * (float)Dh * 1.02f;
  dim3 grid(nsplit, H, B);
  switch (Dh) {
    case 64:
      hipLaunchKernelGGL(k_attn_dec<64>, grid, dim3(AD_THREADS), 0, st, qkv, kc, vc, pos, cs, sn,
                         part, cnt, out, H, max_ctx, window, (int)long_layer, scale, shift, eps,
                         nsplit);
      break;
    case 128:
      hipLaunchKernelGGL(k_attn_dec<128>, grid, dim3(AD_THREADS), 0, st, qkv, kc, vc, pos, cs, sn,
                         part, cnt, out, H, max_ctx, window, (int)long_layer, scale, shift, eps,
                         nsplit);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace ann
