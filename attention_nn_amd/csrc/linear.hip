// Projections y = a @ W^T with W stored (N, K) bf16 (each output row a
// contiguous dot product), fused RMSNorm prologue and the block epilogues.
//
//  * k_gemv: M <= 8 rows (batch-1 / small-batch decode).  HBM-bound on the
//    weight stream: groups of LPR lanes walk one weight row with 16-byte
//    loads, U chunks in flight per lane; the (normalised) activations sit in
//    LDS as bf16 and are read with broadcast.
//  * k_gemm: prefill and large-batch decode on MFMA (v_mfma_f32_16x16x32_bf16),
//    128x128x64 tiles, 4 waves of 64x64, register-prefetched K loop.
#include "common.h"
#include "launch.h"

namespace ann {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

// Epilogue for one output element (row m, column n) of accumulator y.
template <int EPI>
__device__ __forceinline__ void epilogue(const EpiArgs& ea, int m, int n, float y) {
  if (EPI == EPI_STORE) {
    ea.out[(size_t)m * ea.ldo + n] = f2bf(y);
  } else if (EPI == EPI_RELU2) {
    float u = rbf(y);
    float r = u > 0.f ? u : 0.f;
    ea.out[(size_t)m * ea.ldo + n] = f2bf(r * r);
  } else if (EPI == EPI_RESID_ATTN) {
    const size_t i = (size_t)m * ea.ldr + n;
    float yb = rbf(y);
    float t = rbf(rbf(ea.lam[0] * bf2f(ea.x[i])) + rbf(ea.lam[2] * yb));
    ea.x[i] = f2bf(t + rbf(ea.lam[4] * bf2f(ea.x0[i])));
  } else if (EPI == EPI_RESID_MLP) {
    const size_t i = (size_t)m * ea.ldr + n;
    float yb = rbf(y);
    ea.x[i] = f2bf(rbf(ea.lam[1] * bf2f(ea.x[i])) + rbf(ea.lam[3] * yb));
  } else {  // EPI_LOGITS
    const bf16_t z = f2bf(y);
    const size_t i = (size_t)m * ea.ldz + n;
    if (ea.z) ea.z[i] = z;
    if (ea.logits) ea.logits[i] = softcap(bf2f(z));
  }
}

// ---- GEMV -------------------------------------------------------------------

constexpr int GEMV_THREADS = 256;
constexpr int GEMV_U = 4;  // 16-byte weight chunks in flight per lane

template <int M, int LPR, int EPI, bool RMS>
__global__ __launch_bounds__(GEMV_THREADS) void k_gemv(const bf16_t* __restrict__ W,
                                                       const bf16_t* __restrict__ X, int ldx,
                                                       int N, int K, float eps, EpiArgs ea) {
  extern __shared__ uint4 xs4[];                 // M * K bf16, normalised if RMS
  __shared__ float red[M][GEMV_THREADS / 64];
  const int tid = threadIdx.x;
  const int K8 = K >> 3;

  float scale[M];
#pragma unroll
  for (int m = 0; m < M; ++m) scale[m] = 1.f;
  if (RMS) {
    float ss[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      ss[m] = 0.f;
      for (int c = tid; c < K8; c += GEMV_THREADS) {
        float f[8];
        unpack8(*(const uint4*)(X + (size_t)m * ldx + c * 8), f);
#pragma unroll
        for (int j = 0; j < 8; ++j) ss[m] += f[j] * f[j];
      }
      ss[m] = group_sum<64>(ss[m]);
      if ((tid & 63) == 0) red[m][tid >> 6] = ss[m];
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < GEMV_THREADS / 64; ++w) t += red[m][w];
      scale[m] = rsqrtf(t / (float)K + eps);
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m) {
    for (int c = tid; c < K8; c += GEMV_THREADS) {
      uint4 v = *(const uint4*)(X + (size_t)m * ldx + c * 8);
      if (RMS) {
        float f[8];
        unpack8(v, f);
        v.x = pack2(f[0] * scale[m], f[1] * scale[m]);
        v.y = pack2(f[2] * scale[m], f[3] * scale[m]);
        v.z = pack2(f[4] * scale[m], f[5] * scale[m]);
        v.w = pack2(f[6] * scale[m], f[7] * scale[m]);
      }
      xs4[m * K8 + c] = v;
    }
  }
  __syncthreads();

  constexpr int G = GEMV_THREADS / LPR;
  const int g = tid / LPR, lig = tid % LPR;
  const int n = blockIdx.x * G + g;
  const bool live = n < N;
  const uint4* wrow = (const uint4*)(W + (size_t)(live ? n : 0) * K);
  float acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.f;

  for (int c0 = 0; c0 < K8; c0 += LPR * GEMV_U) {
    uint4 w[GEMV_U];
#pragma unroll
    for (int u = 0; u < GEMV_U; ++u) {
      const int c = c0 + u * LPR + lig;
      w[u] = (live && c < K8) ? wrow[c] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < GEMV_U; ++u) {
      const int c = c0 + u * LPR + lig;
      if (c < K8) {
        float wf[8];
        unpack8(w[u], wf);
#pragma unroll
        for (int m = 0; m < M; ++m) {
          float xf[8];
          unpack8(xs4[m * K8 + c], xf);
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[m] += wf[j] * xf[j];
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = group_sum<LPR>(acc[m]);
  if (live) {
#pragma unroll
    for (int m = 0; m < M; ++m)
      if (lig == m) epilogue<EPI>(ea, m, n, acc[m]);
  }
}

bool gemv_fits(int M, int K) {
  return M >= 1 && M <= 8 && (size_t)M * K * 2 <= 64 * 1024 && K % 8 == 0;
}

template <int M, int LPR, int EPI, bool RMS>
static hipError_t launch_gemv(const bf16_t* W, const bf16_t* X, int ldx, int N, int K, float eps,
                              const EpiArgs& ea, hipStream_t st) {
  constexpr int G = GEMV_THREADS / LPR;
  dim3 grid((N + G - 1) / G);
  size_t lds = (size_t)M * K * 2;
  hipLaunchKernelGGL((k_gemv<M, LPR, EPI, RMS>), grid, dim3(GEMV_THREADS), lds, st, W, X, ldx, N,
                     K, eps, ea);
  return hipGetLastError();
}

template <int M, int EPI, bool RMS>
static hipError_t gemv_lpr(const bf16_t* W, const bf16_t* X, int ldx, int N, int K, float eps,
                           const EpiArgs& ea, hipStream_t st) {
  if (K <= 1024) return launch_gemv<M, 32, EPI, RMS>(W, X, ldx, N, K, eps, ea, st);
  return launch_gemv<M, 64, EPI, RMS>(W, X, ldx, N, K, eps, ea, st);
}

template <int M>
static hipError_t gemv_m(int epi, bool rms, const bf16_t* W, const bf16_t* X, int ldx, int N,
                         int K, float eps, const EpiArgs& ea, hipStream_t st) {
  switch (epi) {
    case EPI_STORE:
      return rms ? gemv_lpr<M, EPI_STORE, true>(W, X, ldx, N, K, eps, ea, st)
                 : gemv_lpr<M, EPI_STORE, false>(W, X, ldx, N, K, eps, ea, st);
    case EPI_RELU2:
      return rms ? gemv_lpr<M, EPI_RELU2, true>(W, X, ldx, N, K, eps, ea, st)
                 : gemv_lpr<M, EPI_RELU2, false>(W, X, ldx, N, K, eps, ea, st);
    case EPI_RESID_ATTN:
      return gemv_lpr<M, EPI_RESID_ATTN, false>(W, X, ldx, N, K, eps, ea, st);
    case EPI_RESID_MLP:
      return gemv_lpr<M, EPI_RESID_MLP, false>(W, X, ldx, N, K, eps, ea, st);
    case EPI_LOGITS:
      return rms ? gemv_lpr<M, EPI_LOGITS, true>(W, X, ldx, N, K, eps, ea, st)
                 : gemv_lpr<M, EPI_LOGITS, false>(W, X, ldx, N, K, eps, ea, st);
  }
  return hipErrorInvalidValue;
}

hipError_t gemv(int epi, bool rms_in, const bf16_t* W, const bf16_t* X, int ldx, int M, int N,
                int K, float eps, const EpiArgs& ea, hipStream_t st) {
  if (!gemv_fits(M, K)) return hipErrorInvalidValue;
  switch (M) {
    case 1: return gemv_m<1>(epi, rms_in, W, X, ldx, N, K, eps, ea, st);
    case 2: return gemv_m<2>(epi, rms_in, W, X, ldx, N, K, eps, ea, st);
    case 3: return gemv_m<3>(epi, rms_in, W, X, ldx, N, K, eps, ea, st);
    case 4: return gemv_m<4>(epi, rms_in, W, X, ldx, N, K, eps, ea, st);
    case 5: return gemv_m<5>(epi, rms_in, W, X, ldx, N, K, eps, ea, st);
    case 6: return gemv_m<6>(epi, rms_in, W, X, ldx, N, K, eps, ea, st);
    case 7: return gemv_m<7>(epi, rms_in, W, X, ldx, N, K, eps, ea, st);
    case 8: return gemv_m<8>(epi, rms_in, W, X, ldx, N, K, eps, ea, st);
  }
  return hipErrorInvalidValue;
}

// ---- MFMA GEMM --------------------------------------------------------------

constexpr int GM_BM = 128, GM_BN = 128, GM_BK = 64, GM_LDS = GM_BK + 8;  // +16 B row pad

template <int EPI>
__global__ __launch_bounds__(256) void k_gemm(const bf16_t* __restrict__ A, int lda,
                                              const float* __restrict__ rs,
                                              const bf16_t* __restrict__ W, int M, int N, int K,
                                              EpiArgs ea) {
  __shared__ __attribute__((aligned(16))) bf16_t As[GM_BM * GM_LDS];
  __shared__ __attribute__((aligned(16))) bf16_t Bs[GM_BN * GM_LDS];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv >> 1, wn = wv & 1;
  const int m0 = blockIdx.y * GM_BM, n0 = blockIdx.x * GM_BN;

  // each thread moves 4 16-byte chunks of A and 4 of B per K tile
  int arow[4], acol[4];
  float ascale[4];
  bool aok[4], bok[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int id = tid + i * 256;
    arow[i] = id >> 3;
    acol[i] = (id & 7) * 8;
    aok[i] = (m0 + arow[i]) < M;
    bok[i] = (n0 + arow[i]) < N;
    ascale[i] = (rs && aok[i]) ? rs[m0 + arow[i]] : 1.f;
  }
  uint4 ra[4], rb[4];
  auto load_tile = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ra[i] = aok[i] ? *(const uint4*)(A + (size_t)(m0 + arow[i]) * lda + k0 + acol[i])
                     : make_uint4(0, 0, 0, 0);
      rb[i] = bok[i] ? *(const uint4*)(W + (size_t)(n0 + arow[i]) * K + k0 + acol[i])
                     : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint4 v = ra[i];
      if (rs) {
        float f[8];
        unpack8(v, f);
        const float s = ascale[i];
        v.x = pack2(f[0] * s, f[1] * s);
        v.y = pack2(f[2] * s, f[3] * s);
        v.z = pack2(f[4] * s, f[5] * s);
        v.w = pack2(f[6] * s, f[7] * s);
      }
      *(uint4*)(As + arow[i] * GM_LDS + acol[i]) = v;
      *(uint4*)(Bs + arow[i] * GM_LDS + acol[i]) = rb[i];
    }
  };

  floatx4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (floatx4_t){0.f, 0.f, 0.f, 0.f};

  const int r16 = lane & 15, kq = (lane >> 4) * 8;
  load_tile(0);
  for (int k0 = 0; k0 < K; k0 += GM_BK) {
    __syncthreads();
    store_tile();
    __syncthreads();
    if (k0 + GM_BK < K) load_tile(k0 + GM_BK);
#pragma unroll
    for (int kk = 0; kk < GM_BK; kk += 32) {
      bf16x8_t a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        a[i] = *(const bf16x8_t*)(As + (wm * 64 + i * 16 + r16) * GM_LDS + kk + kq);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        b[j] = *(const bf16x8_t*)(Bs + (wn * 64 + j * 16 + r16) * GM_LDS + kk + kq);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  }
  // C layout of 16x16 MFMA: lane holds column (lane & 15), rows 4*(lane>>4) + r
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + wn * 64 + j * 16 + r16;
      if (n >= N) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + r;
        if (m < M) epilogue<EPI>(ea, m, n, acc[i][j][r]);
      }
    }
}

hipError_t gemm(int epi, const bf16_t* A, int lda, const float* rs, const bf16_t* W, int M, int N,
                int K, const EpiArgs& ea, hipStream_t st) {
  if (K % GM_BK != 0 || M <= 0 || N <= 0) return hipErrorInvalidValue;
  dim3 grid((N + GM_BN - 1) / GM_BN, (M + GM_BM - 1) / GM_BM);
  switch (epi) {
    case EPI_STORE:
      hipLaunchKernelGGL(k_gemm<EPI_STORE>, grid, dim3(256), 0, st, A, lda, rs, W, M, N, K, ea);
      break;
    case EPI_RELU2:
      hipLaunchKernelGGL(k_gemm<EPI_RELU2>, grid, dim3(256), 0, st, A, lda, rs, W, M, N, K, ea);
      break;
    case EPI_RESID_ATTN:
      hipLaunchKernelGGL(k_gemm<EPI_RESID_ATTN>, grid, dim3(256), 0, st, A, lda, rs, W, M, N, K, ea);
      break;
    case EPI_RESID_MLP:
      hipLaunchKernelGGL(k_gemm<EPI_RESID_MLP>, grid, dim3(256), 0, st, A, lda, rs, W, M, N, K, ea);
      break;
    case EPI_LOGITS:
      hipLaunchKernelGGL(k_gemm<EPI_LOGITS>, grid, dim3(256), 0, st, A, lda, rs, W, M, N, K, ea);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace ann
