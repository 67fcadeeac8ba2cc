// Element-wise and row kernels: weight packing, RoPE tables, embedding +
// RMSNorm, QK-norm + RoPE + KV-cache append, and the operator entry points
// (relu2, rope_ht, rms_norm) that mirror the reference's Metal kernels.
#include "common.h"
#include "launch.h"

namespace ann {

// ---- weight packing ---------------------------------------------------------

// dst (N, K) bf16 row-major  <-  src (K, N) fp32 row-major (the reference's
// (in, out) storage), value bf16(bf16(w) * bf16(scale)) when scale_ptr is set
// (model.py:239-241: weights cast to bf16, then multiplied by a bf16 lambda),
// plain bf16(w) otherwise.  32x32 tiles through LDS so both sides coalesce.
__global__ void k_pack_transpose(const float* __restrict__ src, bf16_t* __restrict__ dst,
                                 int K, int N, int ldd, const float* __restrict__ scale_ptr) {
  __shared__ float tile[32][33];
  const int n0 = blockIdx.x * 32, k0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 256 threads: 32 x 8
  for (int r = ty; r < 32; r += 8) {
    int k = k0 + r, n = n0 + tx;
    tile[r][tx] = (k < K && n < N) ? src[(size_t)k * N + n] : 0.f;
  }
  __syncthreads();
  const float s = scale_ptr ? rbf(*scale_ptr) : 1.f;
  for (int r = ty; r < 32; r += 8) {
    int n = n0 + r, k = k0 + tx;
    if (n < N && k < K) {
      float w = rbf(tile[tx][r]);
      dst[(size_t)n * ldd + k] = f2bf(scale_ptr ? w * s : w);
    }
  }
}

// Same-layout fp32 -> bf16 copy (embedding rows).
__global__ void k_pack_cast(const float* __restrict__ src, bf16_t* __restrict__ dst, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) dst[i] = f2bf(src[i]);
}

// Per-layer lambdas, bf16-rounded (model.py:229-232): row l = r0 r1 p0 p1 x0.
__global__ void k_pack_lambdas(const float* resid, const float* post, const float* x0l,
                               float* out, int L) {
  int l = blockIdx.x * blockDim.x + threadIdx.x;
  if (l >= L) return;
  float* o = out + l * 8;
  o[0] = rbf(resid[2 * l]);
  o[1] = rbf(resid[2 * l + 1]);
  o[2] = rbf(post[2 * l]);
  o[3] = rbf(post[2 * l + 1]);
  o[4] = rbf(x0l[l]);
  o[5] = o[6] = o[7] = 0.f;
}

// RoPE tables (metal_kernels.py:144-150): freq_i = (1/base)^(i/(D/4-1)),
// theta = t * freq_i, fp32 cos / sin.
__global__ void k_rope_tables(float* cs, float* sn, int seq_len, int d4, float base) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= seq_len * d4) return;
  int t = i / d4, j = i % d4;
  float lin = d4 > 1 ? (float)j / (float)(d4 - 1) : 0.f;
  float freq = powf(1.0f / base, lin);
  float th = (float)t * freq;
  cs[i] = cosf(th);
  sn[i] = sinf(th);
}

// ---- embedding + RMSNorm ------------------------------------------------------

// x = x0 = rms(bf16(embed[tok])) (model.py:236-237).  One block per row.
__global__ void k_embed_rms(const int32_t* __restrict__ tok, const bf16_t* __restrict__ emb,
                            bf16_t* __restrict__ x, bf16_t* __restrict__ x0, int d, int V,
                            float eps) {
  __shared__ float red[16];
  const int m = blockIdx.x;
  int t = tok[m];
  t = t < 0 ? 0 : (t >= V ? V - 1 : t);   // host validates; clamp keeps reads in bounds
  const bf16_t* e = emb + (size_t)t * d;
  float ss = 0.f;
  for (int i = threadIdx.x; i < d; i += blockDim.x) {
    float v = bf2f(e[i]);
    ss += v * v;
  }
  float s = rsqrtf(block_sum(ss, red) / (float)d + eps);
  for (int i = threadIdx.x; i < d; i += blockDim.x) {
    bf16_t r = f2bf(bf2f(e[i]) * s);
    x[(size_t)m * d + i] = r;
    x0[(size_t)m * d + i] = r;
  }
}

// h = bf16(x * rsqrt(mean(x^2) + eps)) (model.py:49 with the bf16 output of
// an eager op); one work-group per row, every chunk loaded up front.
__global__ __launch_bounds__(256) void k_rms_apply(const bf16_t* __restrict__ x, int ldx,
                                                   bf16_t* __restrict__ h, int ldh, int d,
                                                   float eps) {
  __shared__ float red[4];
  const int m = blockIdx.x, tid = threadIdx.x;
  const uint4* r = (const uint4*)(x + (size_t)m * ldx);
  uint4* o = (uint4*)(h + (size_t)m * ldh);
  const int K8 = d >> 3;
  uint4 v[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int c = tid + u * 256;
    v[u] = c < K8 ? r[c] : make_uint4(0, 0, 0, 0);
  }
  float ss = 0.f;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    float f[8];
    unpack8(v[u], f);
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += f[j] * f[j];
  }
  const float s = rsqrtf(block_sum(ss, red) / (float)d + eps);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int c = tid + u * 256;
    if (c < K8) {
      float f[8];
      unpack8(v[u], f);
      uint4 w;
      w.x = pack2(f[0] * s, f[1] * s);
      w.y = pack2(f[2] * s, f[3] * s);
      w.z = pack2(f[4] * s, f[5] * s);
      w.w = pack2(f[6] * s, f[7] * s);
      o[c] = w;
    }
  }
}

// The same with one wave per row (CPL 16-byte chunks per lane, d <= 512 CPL)
// and four rows per work-group: the row sum is a wave reduction, no barrier.
// One work-group per row left 160 of 256 threads idle at d = 768 and made
// every row pay a barrier: 26.8 us for 32768 rows, a 100 MB round trip.
template <int CPL>
__global__ __launch_bounds__(256) void k_rms_rows(const bf16_t* __restrict__ x, int ldx,
                                                  bf16_t* __restrict__ h, int ldh, int M, int d,
                                                  float eps) {
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= M) return;
  const uint4* r = (const uint4*)(x + (size_t)m * ldx);
  uint4* o = (uint4*)(h + (size_t)m * ldh);
  const int K8 = d >> 3;
  uint4 v[CPL];
#pragma unroll
  for (int u = 0; u < CPL; ++u) {
    const int c = lane + u * 64;
    v[u] = c < K8 ? r[c] : make_uint4(0, 0, 0, 0);
  }
  float ss = 0.f;
#pragma unroll
  for (int u = 0; u < CPL; ++u) {
    float f[8];
    unpack8(v[u], f);
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += f[j] * f[j];
  }
  const float s = rsqrtf(wave_sum(ss) / (float)d + eps);
#pragma unroll
  for (int u = 0; u < CPL; ++u) {
    const int c = lane + u * 64;
    if (c < K8) {
      float f[8];
      unpack8(v[u], f);
      uint4 w;
      w.x = pack2(f[0] * s, f[1] * s);
      w.y = pack2(f[2] * s, f[3] * s);
      w.z = pack2(f[4] * s, f[5] * s);
      w.w = pack2(f[6] * s, f[7] * s);
      o[c] = w;
    }
  }
}

// ---- QK-norm + RoPE + KV-cache append --------------------------------------

// qkv (M, 3*H*Dh) bf16 -> q (M, H*Dh) = rope(rms(q)); K/V cache rows written
// at the token's position (model.py:244-247).  Row m is token t = m % T of
// sequence b = m / T at position pos[b] + t.  Cache layout [b][h][ctx][Dh].
// One group of Dh/2 lanes per (row, head); each lane owns one dim pair.
template <int DH>
__global__ void k_qkv_post(const bf16_t* __restrict__ qkv, bf16_t* __restrict__ q,
                           bf16_t* __restrict__ kc, bf16_t* __restrict__ vc,
                           const int32_t* __restrict__ pos, const float* __restrict__ cs,
                           const float* __restrict__ sn, int M, int T, int H, int max_ctx,
                           float eps) {
  constexpr int P = DH / 2;                  // lanes per head
  constexpr int D4 = DH / 4;
  const int gid = blockIdx.x * (blockDim.x / P) + threadIdx.x / P;
  const int p = threadIdx.x % P;
  if (gid >= M * H) return;
  const int m = gid / H, h = gid % H;
  const int b = m / T, t = m % T;
  const int ps = pos[b] + t;
  const int d = H * DH;
  const bf16_t* row = qkv + (size_t)m * 3 * d;
  const uint32_t qw = *(const uint32_t*)(row + h * DH + 2 * p);
  const uint32_t kw = *(const uint32_t*)(row + d + h * DH + 2 * p);
  const uint32_t vw = *(const uint32_t*)(row + 2 * d + h * DH + 2 * p);
  float q0 = __uint_as_float(qw << 16), q1 = __uint_as_float(qw & 0xffff0000u);
  float k0 = __uint_as_float(kw << 16), k1 = __uint_as_float(kw & 0xffff0000u);
  float sq = group_sum<P>(q0 * q0 + q1 * q1);
  float sk = group_sum<P>(k0 * k0 + k1 * k1);
  float rq = rsqrtf(sq / (float)DH + eps), rk = rsqrtf(sk / (float)DH + eps);
  q0 = rbf(q0 * rq); q1 = rbf(q1 * rq);
  k0 = rbf(k0 * rk); k1 = rbf(k1 * rk);
  if (p < D4) {
    const float c = cs[ps * D4 + p], s = sn[ps * D4 + p];
    float a0 = c * q0 + s * q1, a1 = c * q1 - s * q0;
    float b0 = c * k0 + s * k1, b1 = c * k1 - s * k0;
    q0 = a0; q1 = a1; k0 = b0; k1 = b1;
  }
  *(uint32_t*)(q + (size_t)m * d + h * DH + 2 * p) = pack2(q0, q1);
  const size_t cidx = (((size_t)b * H + h) * max_ctx + ps) * DH + 2 * p;
  *(uint32_t*)(kc + cidx) = pack2(k0, k1);
  *(uint32_t*)(vc + cidx) = vw;
}

// ---- softcapped cross-entropy: per-row loss and the mean --------------------
//
// ce_softcap_fwd (metal_kernels.py:153-193) after the lm_head GEMM has left,
// per 128-column tile t and row m, the partial sum of exp(softcap(z)) in
// part[t * ld + m] and the target's softcapped logit in tz[m]:
//   loss[m] = log(sum_t part[t][m]) - tz[m]
// A work-group takes 64 rows (one per lane, coalesced across the wave); its
// four waves each sum a contiguous quarter of the tiles, and the quarters are
// added in wave order.  The mean (model.py:221) is one work-group summing the
// rows in a fixed order.
constexpr int CE_ROWS = 64;

__global__ __launch_bounds__(256) void k_ce_rows(const float* __restrict__ part, int ld,
                                                 int ntiles, const float* __restrict__ tz, int M,
                                                 float* __restrict__ rows) {
  __shared__ float q[4][CE_ROWS];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int m = blockIdx.x * CE_ROWS + lane;
  const int per = (ntiles + 3) / 4;
  const int t0 = wv * per, t1 = min(ntiles, t0 + per);
  float sum = 0.f;
  if (m < M) {
    const float* p = part + m;
    int t = t0;
    for (; t + 8 <= t1; t += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = p[(size_t)(t + u) * ld];
#pragma unroll
      for (int u = 0; u < 8; ++u) sum += v[u];
    }
    for (; t < t1; ++t) sum += p[(size_t)t * ld];
  }
  q[wv][lane] = sum;
  __syncthreads();
  if (wv == 0 && m < M) rows[m] = logf(((q[0][lane] + q[1][lane]) + q[2][lane]) + q[3][lane]) - tz[m];
}

constexpr int CE_MEAN_THREADS = 1024;

__global__ __launch_bounds__(CE_MEAN_THREADS) void k_ce_mean(const float* __restrict__ rows, int M,
                                                            float* __restrict__ mean) {
  __shared__ float buf[CE_MEAN_THREADS];
  const int tid = threadIdx.x;
  float sum = 0.f;
  for (int m = tid; m < M; m += CE_MEAN_THREADS) sum += rows[m];
  buf[tid] = sum;
  __syncthreads();
  for (int w = CE_MEAN_THREADS / 2; w > 0; w >>= 1) {
    if (tid < w) buf[tid] += buf[tid + w];
    __syncthreads();
  }
  if (tid == 0) *mean = buf[0] / (float)M;
}

// ---- operators (reference kernel API) ----------------------------------------

template <typename T> __device__ __forceinline__ float ldf(const T* p, size_t i);
template <> __device__ __forceinline__ float ldf<float>(const float* p, size_t i) { return p[i]; }
template <> __device__ __forceinline__ float ldf<bf16_t>(const bf16_t* p, size_t i) { return bf2f(p[i]); }
template <typename T> __device__ __forceinline__ void stf(T* p, size_t i, float v);
template <> __device__ __forceinline__ void stf<float>(float* p, size_t i, float v) { p[i] = v; }
template <> __device__ __forceinline__ void stf<bf16_t>(bf16_t* p, size_t i, float v) { p[i] = f2bf(v); }

// relu2 (metal_kernels.py:37-47): y = (T)(max(x,0)^2), fp32 inside.
template <typename T>
__global__ void k_relu2(const T* __restrict__ x, T* __restrict__ y, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) {
    float v = ldf(x, i);
    float r = v > 0.f ? v : 0.f;
    stf(y, i, r * r);
  }
}

// rope_ht (metal_kernels.py:87-134 semantics): each head vector of D elements
// is rotated in adjacent pairs, pair j < D/4 by the angle of table index j at
// position pos0 + t, pairs j >= D/4 passed through.  One wave per (row, head)
// vector, four vectors per 256-thread work-group; lane l moves pairs l,
// l + 64, ..  (as one 8-byte / 4-byte word where x and y allow, VEC).  The
// inverse rotation is the forward one with the sine negated.
template <typename T> struct RopePair;
template <> struct RopePair<float> {
  typedef float2 W;
  static __device__ __forceinline__ void get(W w, float& a, float& b) { a = w.x; b = w.y; }
  static __device__ __forceinline__ W put(float a, float b) { return make_float2(a, b); }
};
template <> struct RopePair<bf16_t> {
  typedef uint32_t W;
  static __device__ __forceinline__ void get(W w, float& a, float& b) {
    a = __uint_as_float(w << 16);
    b = __uint_as_float(w & 0xffff0000u);
  }
  static __device__ __forceinline__ W put(float a, float b) { return pack2(a, b); }
};

template <typename T, bool VEC>
__global__ __launch_bounds__(256) void k_rope(const T* __restrict__ x, T* __restrict__ y,
                                              const float* __restrict__ cs,
                                              const float* __restrict__ sn, long long nvec, int Tn,
                                              int H, int D, int pos0, float sgn) {
  const long long v = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (v >= nvec) return;
  const int lane = threadIdx.x & 63, nrot = D / 4;
  const size_t tab = (size_t)((int)((v / H) % Tn) + pos0) * nrot;
  const T* xv = x + (size_t)v * D;
  T* yv = y + (size_t)v * D;
  for (int j = lane; j < D / 2; j += 64) {
    float a, b;
    if constexpr (VEC) {
      RopePair<T>::get(((const typename RopePair<T>::W*)xv)[j], a, b);
    } else {
      a = ldf(xv, 2 * j);
      b = ldf(xv, 2 * j + 1);
    }
    if (j < nrot) {
      const float c = cs[tab + j], s = sgn * sn[tab + j];
      const float ra = c * a + s * b, rb = c * b - s * a;
      a = ra;
      b = rb;
    }
    if constexpr (VEC) {
      ((typename RopePair<T>::W*)yv)[j] = RopePair<T>::put(a, b);
    } else {
      stf(yv, 2 * j, a);
      stf(yv, 2 * j + 1, b);
    }
  }
}

// rms (model.py:48-49) over rows; one block per row.
template <typename T>
__global__ void k_rms(const T* __restrict__ x, T* __restrict__ y, int dim, float eps) {
  __shared__ float red[16];
  const T* r = x + (size_t)blockIdx.x * dim;
  T* o = y + (size_t)blockIdx.x * dim;
  float ss = 0.f;
  for (int i = threadIdx.x; i < dim; i += blockDim.x) {
    float v = ldf(r, i);
    ss += v * v;
  }
  float s = rsqrtf(block_sum(ss, red) / (float)dim + eps);
  for (int i = threadIdx.x; i < dim; i += blockDim.x) stf(o, i, ldf(r, i) * s);
}

// ---- launchers ---------------------------------------------------------------

static inline unsigned cdiv(size_t a, size_t b) { return (unsigned)((a + b - 1) / b); }

hipError_t pack_transpose(const float* src, bf16_t* dst, int K, int N, int ldd,
                          const float* scale, hipStream_t st) {
  dim3 g(cdiv(N, 32), cdiv(K, 32));
  hipLaunchKernelGGL(k_pack_transpose, g, dim3(256), 0, st, src, dst, K, N, ldd, scale);
  return hipGetLastError();
}

hipError_t pack_cast(const float* src, bf16_t* dst, size_t n, hipStream_t st) {
  unsigned g = cdiv(n, 256);
  if (g > 65536) g = 65536;
  hipLaunchKernelGGL(k_pack_cast, dim3(g), dim3(256), 0, st, src, dst, n);
  return hipGetLastError();
}

hipError_t pack_lambdas(const float* resid, const float* post, const float* x0l, float* out,
                        int L, hipStream_t st) {
  hipLaunchKernelGGL(k_pack_lambdas, dim3(cdiv(L, 64)), dim3(64), 0, st, resid, post, x0l, out, L);
  return hipGetLastError();
}

hipError_t rope_tables(float* cs, float* sn, int seq_len, int head_dim, float base,
                       hipStream_t st) {
  int d4 = head_dim / 4;
  hipLaunchKernelGGL(k_rope_tables, dim3(cdiv((size_t)seq_len * d4, 256)), dim3(256), 0, st, cs,
                     sn, seq_len, d4, base);
  return hipGetLastError();
}

hipError_t embed_rms(const int32_t* tok, const bf16_t* emb, bf16_t* x, bf16_t* x0, int M, int d,
                     int V, float eps, hipStream_t st) {
  hipLaunchKernelGGL(k_embed_rms, dim3(M), dim3(256), 0, st, tok, emb, x, x0, d, V, eps);
  return hipGetLastError();
}

hipError_t rms_apply(const bf16_t* x, int ldx, bf16_t* h, int ldh, int M, int d, float eps,
                     hipStream_t st) {
  if (d > 8192 || d % 8) return hipErrorInvalidValue;
  const dim3 g4(cdiv(M, 4));
  if (d <= 1024)
    hipLaunchKernelGGL(k_rms_rows<2>, g4, dim3(256), 0, st, x, ldx, h, ldh, M, d, eps);
  else if (d <= 2048)
    hipLaunchKernelGGL(k_rms_rows<4>, g4, dim3(256), 0, st, x, ldx, h, ldh, M, d, eps);
  else
    hipLaunchKernelGGL(k_rms_apply, dim3(M), dim3(256), 0, st, x, ldx, h, ldh, d, eps);
  return hipGetLastError();
}

hipError_t qkv_post(const bf16_t* qkv, bf16_t* q, bf16_t* kc, bf16_t* vc, const int32_t* pos,
                    const float* cs, const float* sn, int M, int T, int H, int Dh, int max_ctx,
                    float eps, hipStream_t st) {
  const size_t groups = (size_t)M * H;
  switch (Dh) {
#define ANN_QKV_CASE(D)                                                                        \
  case D: {                                                                                    \
    constexpr int per = 256 / (D / 2);                                                         \
    hipLaunchKernelGGL(k_qkv_post<D>, dim3(cdiv(groups, per)), dim3(256), 0, st, qkv, q, kc,   \
                       vc, pos, cs, sn, M, T, H, max_ctx, eps);                                \
    break;                                                                                     \
  }
    ANN_QKV_CASE(32)
    ANN_QKV_CASE(64)
    ANN_QKV_CASE(128)
#undef ANN_QKV_CASE
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t ce_finalize(const float* part, int ld, int ntiles, const float* tz, int M, float* rows,
                       float* mean, hipStream_t st) {
  if (M <= 0 || ntiles <= 0 || ld < M || !part || !tz || !rows || !mean)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_ce_rows, dim3(cdiv(M, CE_ROWS)), dim3(256), 0, st, part, ld, ntiles, tz,
                     M, rows);
  hipLaunchKernelGGL(k_ce_mean, dim3(1), dim3(CE_MEAN_THREADS), 0, st, rows, M, mean);
  return hipGetLastError();
}

hipError_t op_relu2(const void* x, void* y, size_t n, int dtype, hipStream_t st) {
  unsigned g = cdiv(n, 256);
  if (g > 65536) g = 65536;
  if (g == 0) return hipSuccess;
  if (dtype == 0)
    hipLaunchKernelGGL(k_relu2<float>, dim3(g), dim3(256), 0, st, (const float*)x, (float*)y, n);
  else
    hipLaunchKernelGGL(k_relu2<bf16_t>, dim3(g), dim3(256), 0, st, (const bf16_t*)x, (bf16_t*)y, n);
  return hipGetLastError();
}

hipError_t op_rope(const void* x, void* y, const float* cs, const float* sn, int B, int T, int H,
                   int D, int pos0, int inverse, int dtype, hipStream_t st) {
  const long long nvec = (long long)B * T * H;
  if (nvec == 0) return hipSuccess;
  const dim3 grid((unsigned)((nvec + 3) / 4));
  const float sgn = inverse ? -1.f : 1.f;
  // pairs as whole words when both buffers are aligned to a pair
  const uintptr_t pa = (dtype == 0 ? 8 : 4) - 1;
  const bool vec = (((uintptr_t)x | (uintptr_t)y) & pa) == 0;
#define ANN_ROPE(TY, V)                                                                       \
  hipLaunchKernelGGL((k_rope<TY, V>), grid, dim3(256), 0, st, (const TY*)x, (TY*)y, cs, sn, nvec, \
                     T, H, D, pos0, sgn)
  if (dtype == 0) {
    if (vec) ANN_ROPE(float, true); else ANN_ROPE(float, false);
  } else {
    if (vec) ANN_ROPE(bf16_t, true); else ANN_ROPE(bf16_t, false);
  }
#undef ANN_ROPE
  return hipGetLastError();
}

hipError_t op_rms(const void* x, void* y, int rows, int dim, float eps, int dtype, hipStream_t st) {
  if (rows == 0) return hipSuccess;
  if (dtype == 0)
    hipLaunchKernelGGL(k_rms<float>, dim3(rows), dim3(256), 0, st, (const float*)x, (float*)y, dim, eps);
  else
    hipLaunchKernelGGL(k_rms<bf16_t>, dim3(rows), dim3(256), 0, st, (const bf16_t*)x, (bf16_t*)y, dim, eps);
  return hipGetLastError();
}

}  // namespace ann
