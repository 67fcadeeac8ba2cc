// Projections y = a @ W^T with W stored (N, K) bf16 (each output row a
// contiguous dot product), fused RMSNorm prologue and the block epilogues.
//
//  * k_gemv: M <= 8 rows (batch-1 / small-batch decode).  HBM-bound on the
//    weight stream: groups of LPR lanes walk one weight row with 16-byte
//    loads, U chunks in flight per lane; the (normalised) activations sit in
//    LDS as bf16 and are read with broadcast.
//  * k_gemm_sk / k_gemm_sk2: decode projections for 8 < M <= 128 rows on
//    MFMA, one 16x16 or 32x32 output tile per work-group, K split over the
//    four waves.
//  * k_gemm / k_gemm_2w / k_gemm_bat: prefill, wide outputs and batched
//    products on MFMA (v_mfma_f32_16x16x32_bf16): 64..256 x 128..256 x 64
//    tiles of four waves, swizzled LDS, register-prefetched K loop.
#include <stdlib.h>
#include <type_traits>
#include "common.h"
#include "launch.h"
#include "epilogue.h"
#include "sk_gemm.h"

namespace ann {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
// register-ring element: a native vector (an array of HIP's uint4 struct that
// stays live across loop iterations is kept in scratch memory, not registers)
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// f(integral_constant<int, I>) for I = I .. N-1: the slots of a register ring
// indexed by compile-time constants
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// Epilogue for one output element (row m, column n) of accumulator y.
template <int EPI>
__device__ __forceinline__ void epilogue(const EpiArgs& ea, int m, int n, float y) {
  if (EPI == EPI_STORE) {
    ea.out[(size_t)m * ea.ldo + n] = f2bf(y);
  } else if (EPI == EPI_RELU2) {
    ea.out[(size_t)m * ea.ldo + n] = relu2_bf(y);
  } else if (EPI == EPI_RESID_ATTN) {
    const size_t i = (size_t)m * ea.ldr + n;
    ea.x[i] = mix_attn(ea.lam, bf2f(ea.x[i]), bf2f(ea.x0[i]), y);
  } else if (EPI == EPI_RESID_MLP) {
    const size_t i = (size_t)m * ea.ldr + n;
    ea.x[i] = mix_mlp(ea.lam, bf2f(ea.x[i]), y);
  } else if (EPI == EPI_PE_B) {
    const size_t i = (size_t)m * ea.ldr + n;
    ea.out[(size_t)m * ea.ldo + n] = f2bf(rbf(ea.s0 * bf2f(ea.x[i])) + rbf(ea.s1 * rbf(y)));
  } else if (EPI == EPI_PE_X) {
    const size_t i = (size_t)m * ea.ldr + n;
    const bf16_t o = f2bf(rbf(ea.s0 * bf2f(ea.x[i])) + rbf(y));
    ea.out[(size_t)m * ea.ldo + n] = o;
    if (ea.outT) ea.outT[(size_t)n * ea.ldoT + m] = o;
  } else {  // EPI_LOGITS
    const bf16_t z = f2bf(y);
    const size_t i = (size_t)m * ea.ldz + n;
    if (ea.z) ea.z[i] = z;
    if (ea.logits) ea.logits[i] = softcap(bf2f(z));
  }
}

// Epilogue for the four consecutive columns n..n+3 of row m: one 8-byte
// access per operand (16 bytes for fp32 logits) when all four columns exist
// and the strides and bases keep the accesses aligned, else per element.
template <int EPI>
__device__ __forceinline__ bool epi_vec_ok(const EpiArgs& ea) {
  if (EPI == EPI_STORE || EPI == EPI_RELU2)
    return (ea.ldo & 3) == 0 && ((uintptr_t)ea.out & 7) == 0;
  if (EPI == EPI_RESID_ATTN)
    return (ea.ldr & 3) == 0 && (((uintptr_t)ea.x | (uintptr_t)ea.x0) & 7) == 0;
  if (EPI == EPI_RESID_MLP) return (ea.ldr & 3) == 0 && ((uintptr_t)ea.x & 7) == 0;
  if (EPI == EPI_PE_B || EPI == EPI_PE_X)
    return ((ea.ldr | ea.ldo) & 3) == 0 && (((uintptr_t)ea.x | (uintptr_t)ea.out) & 7) == 0;
  return (ea.ldz & 3) == 0 && ((uintptr_t)ea.z & 7) == 0 && ((uintptr_t)ea.logits & 15) == 0;
}

template <int EPI>
__device__ __forceinline__ void epilogue4(const EpiArgs& ea, bool vec, int m, int n, int N,
                                          const floatx4_t& y) {
  if (!vec || n + 3 >= N) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (n + r < N) epilogue<EPI>(ea, m, n + r, y[r]);
    return;
  }
  if (EPI == EPI_STORE) {
    *(uint2*)(ea.out + (size_t)m * ea.ldo + n) = make_uint2(pack2(y[0], y[1]), pack2(y[2], y[3]));
  } else if (EPI == EPI_RELU2) {
    const uint32_t a = relu2_bf(y[0]) | ((uint32_t)relu2_bf(y[1]) << 16);
    const uint32_t b = relu2_bf(y[2]) | ((uint32_t)relu2_bf(y[3]) << 16);
    *(uint2*)(ea.out + (size_t)m * ea.ldo + n) = make_uint2(a, b);
  } else if (EPI == EPI_RESID_ATTN || EPI == EPI_RESID_MLP) {
    const size_t i = (size_t)m * ea.ldr + n;
    const uint2 xv = *(const uint2*)(ea.x + i);
    const float xf[4] = {__uint_as_float(xv.x << 16), __uint_as_float(xv.x & 0xffff0000u),
                         __uint_as_float(xv.y << 16), __uint_as_float(xv.y & 0xffff0000u)};
    bf16_t o[4];
    if (EPI == EPI_RESID_ATTN) {
      const uint2 zv = *(const uint2*)(ea.x0 + i);
      const float zf[4] = {__uint_as_float(zv.x << 16), __uint_as_float(zv.x & 0xffff0000u),
                           __uint_as_float(zv.y << 16), __uint_as_float(zv.y & 0xffff0000u)};
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = mix_attn(ea.lam, xf[r], zf[r], y[r]);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = mix_mlp(ea.lam, xf[r], y[r]);
    }
    *(uint2*)(ea.x + i) = make_uint2(o[0] | ((uint32_t)o[1] << 16), o[2] | ((uint32_t)o[3] << 16));
  } else if (EPI == EPI_PE_B || EPI == EPI_PE_X) {
    const uint2 xv = *(const uint2*)(ea.x + (size_t)m * ea.ldr + n);
    const float xf[4] = {__uint_as_float(xv.x << 16), __uint_as_float(xv.x & 0xffff0000u),
                         __uint_as_float(xv.y << 16), __uint_as_float(xv.y & 0xffff0000u)};
    float o[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
      o[r] = EPI == EPI_PE_B ? rbf(ea.s0 * xf[r]) + rbf(ea.s1 * rbf(y[r]))
                             : rbf(ea.s0 * xf[r]) + rbf(y[r]);
    *(uint2*)(ea.out + (size_t)m * ea.ldo + n) = make_uint2(pack2(o[0], o[1]), pack2(o[2], o[3]));
    // transposed copy: 2-byte stores, consecutive m across the 16 lanes of a
    // group, so each column's stores coalesce into one 32-byte run
    if (EPI == EPI_PE_X && ea.outT) {
#pragma unroll
      for (int r = 0; r < 4; ++r) ea.outT[(size_t)(n + r) * ea.ldoT + m] = f2bf(o[r]);
    }
  } else {  // EPI_LOGITS
    bf16_t z[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) z[r] = f2bf(y[r]);
    const size_t i = (size_t)m * ea.ldz + n;
    if (ea.z) *(uint2*)(ea.z + i) = make_uint2(z[0] | ((uint32_t)z[1] << 16), z[2] | ((uint32_t)z[3] << 16));
    if (ea.logits)
      *(float4*)(ea.logits + i) = make_float4(softcap(bf2f(z[0])), softcap(bf2f(z[1])),
                                              softcap(bf2f(z[2])), softcap(bf2f(z[3])));
  }
}

// ---- GEMV -------------------------------------------------------------------

constexpr int GEMV_THREADS = 256;

// Fill the LDS activation tile xs (M x K bf16) per the prologue PRE.
template <int M, int PRE>
__device__ __forceinline__ void gemv_prologue(uint4* xs4, const bf16_t* __restrict__ X, int ldx,
                                              int K, float eps, float* red) {
  const int tid = threadIdx.x;
  const int K8 = K >> 3;
  float scale[M];
#pragma unroll
  for (int m = 0; m < M; ++m) scale[m] = 1.f;
  if (PRE == PRE_RMS) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float ss = 0.f;
      for (int c = tid; c < K8; c += GEMV_THREADS) {
        float f[8];
        unpack8(*(const uint4*)(X + (size_t)m * ldx + c * 8), f);
#pragma unroll
        for (int j = 0; j < 8; ++j) ss += f[j] * f[j];
      }
      ss = group_sum<64>(ss);
      if ((tid & 63) == 0) red[m * (GEMV_THREADS / 64) + (tid >> 6)] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < GEMV_THREADS / 64; ++w) t += red[m * (GEMV_THREADS / 64) + w];
      scale[m] = rsqrtf(t / (float)K + eps);
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m) {
    for (int c = tid; c < K8; c += GEMV_THREADS) {
      uint4 v = *(const uint4*)(X + (size_t)m * ldx + c * 8);
      if (PRE == PRE_RMS) {
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
}

template <int M, int LPR, int EPI, int PRE, int GEMV_U>
__global__ __launch_bounds__(GEMV_THREADS) void k_gemv(const bf16_t* __restrict__ W,
                                                       const bf16_t* __restrict__ X, int ldx,
                                                       int N, int K, float eps, EpiArgs ea) {
  extern __shared__ uint4 xs4[];                 // M * K bf16 activations
  constexpr int G = GEMV_THREADS / LPR;          // weight rows per work-group
  __shared__ float red[M * (GEMV_THREADS / 64)];
  __shared__ unsigned long long s_key[G][M];
  const int tid = threadIdx.x;
  const int K8 = K >> 3;

  const int g = tid / LPR, lig = tid % LPR;
  const int n = blockIdx.x * G + g;
  const bool live = n < N;
  const uint4* wrow = (const uint4*)(W + (size_t)(live ? n : 0) * K);
  float acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.f;

  // the first GEMV_U weight chunks of this lane do not depend on the
  // activations: issue them before the prologue so both latencies overlap
  uint4 w[GEMV_U];
#pragma unroll
  for (int u = 0; u < GEMV_U; ++u) {
    const int c = u * LPR + lig;
    w[u] = (live && c < K8) ? wrow[c] : make_uint4(0, 0, 0, 0);
  }
  gemv_prologue<M, PRE>(xs4, X, ldx, K, eps, red);
  __syncthreads();

  for (int c0 = 0; c0 < K8; c0 += LPR * GEMV_U) {
    if (c0) {
#pragma unroll
      for (int u = 0; u < GEMV_U; ++u) {
        const int c = c0 + u * LPR + lig;
        w[u] = (live && c < K8) ? wrow[c] : make_uint4(0, 0, 0, 0);
      }
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
  if (EPI == EPI_LOGITS && ea.amax) {
    // greedy: per-row max of (z, lowest index) over this work-group's rows,
    // stored to amax[m * gridDim.x + block]; k_argmax_finalize reduces them.
#pragma unroll
    for (int m = 0; m < M; ++m)
      if (lig == m)
        s_key[g][m] = (live && n < ea.Vs)
            ? (((unsigned long long)zkey(f2bf(acc[m])) << 32) | (unsigned long long)(0xffffffffu - (unsigned)n))
            : 0ull;
    __syncthreads();
    if (tid < M) {
      unsigned long long best = 0;
#pragma unroll
      for (int i = 0; i < G; ++i) best = s_key[i][tid] > best ? s_key[i][tid] : best;
      ea.amax[(size_t)tid * gridDim.x + blockIdx.x] = best;
    }
  }
}

// out_tok[m] = index of the largest key of row m (lowest index on ties),
// pos[m] += pos_adv.  One work-group per row.
__global__ __launch_bounds__(1024) void k_argmax_finalize(const unsigned long long* __restrict__ keys,
                                                          int nkeys, int32_t* __restrict__ out_tok,
                                                          int32_t* __restrict__ pos, int pos_adv) {
  __shared__ unsigned long long red[16];
  const int m = blockIdx.x, tid = threadIdx.x;
  const unsigned long long* k = keys + (size_t)m * nkeys;
  unsigned long long b0 = 0, b1 = 0, b2 = 0, b3 = 0;
  int i = tid;
  for (; i + 3 * 1024 < nkeys; i += 4 * 1024) {
    const unsigned long long v0 = k[i], v1 = k[i + 1024], v2 = k[i + 2048], v3 = k[i + 3072];
    b0 = v0 > b0 ? v0 : b0;
    b1 = v1 > b1 ? v1 : b1;
    b2 = v2 > b2 ? v2 : b2;
    b3 = v3 > b3 ? v3 : b3;
  }
  for (; i < nkeys; i += 1024) b0 = k[i] > b0 ? k[i] : b0;
  b0 = b1 > b0 ? b1 : b0;
  b2 = b3 > b2 ? b3 : b2;
  unsigned long long best = b2 > b0 ? b2 : b0;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const unsigned lo = __shfl_xor((unsigned)best, o, 64);
    const unsigned hi = __shfl_xor((unsigned)(best >> 32), o, 64);
    const unsigned long long w = ((unsigned long long)hi << 32) | lo;
    best = w > best ? w : best;
  }
  if ((tid & 63) == 0) red[tid >> 6] = best;
  __syncthreads();
  if (tid == 0) {
    unsigned long long b = red[0];
    for (int w = 1; w < 16; ++w) b = red[w] > b ? red[w] : b;
    out_tok[m] = (int32_t)(0xffffffffu - (unsigned)(b & 0xffffffffull));
    if (pos) pos[m] += pos_adv;
  }
}

int gemv_blocks(int N, int K) {
  const int G = GEMV_THREADS / (K <= 1024 ? 32 : 64);
  return (N + G - 1) / G;
}

hipError_t argmax_finalize(const unsigned long long* keys, int nkeys, int M, int32_t* out_tok,
                           int32_t* pos, int pos_adv, hipStream_t st) {
  hipLaunchKernelGGL(k_argmax_finalize, dim3(M), dim3(1024), 0, st, keys, nkeys, out_tok, pos,
                     pos_adv);
  return hipGetLastError();
}

bool gemv_fits(int M, int K) {
  return M >= 1 && M <= 8 && (size_t)M * K * 2 <= 64 * 1024 && K % 8 == 0;
}

// Projections the engine sends to the GEMV: one or two rows.  From four rows
// the skinny MFMA GEMMs are faster (155M decode step, sampled: 4 rows 405.5
// -> 338.2 us, 8 rows 607.3 -> 365.5 us; 2 rows 310.1 on the GEMV against
// 315.1).
bool gemv_routes(int M, int K) { return M <= 2 && gemv_fits(M, K); }

// U = 16-byte weight chunks each lane keeps in flight: enough to hold the
// whole row slice when K / (8 LPR) <= 8, without spilling for short rows.
template <int M, int LPR, int EPI, int PRE>
static hipError_t launch_gemv(const bf16_t* W, const bf16_t* X, int ldx, int N, int K, float eps,
                              const EpiArgs& ea, hipStream_t st) {
  constexpr int G = GEMV_THREADS / LPR;
  dim3 grid((N + G - 1) / G);
  size_t lds = (size_t)M * K * 2;
  if ((K >> 3) <= 4 * LPR)
    hipLaunchKernelGGL((k_gemv<M, LPR, EPI, PRE, 4>), grid, dim3(GEMV_THREADS), lds, st, W, X,
                       ldx, N, K, eps, ea);
  else
    hipLaunchKernelGGL((k_gemv<M, LPR, EPI, PRE, 8>), grid, dim3(GEMV_THREADS), lds, st, W, X,
                       ldx, N, K, eps, ea);
  return hipGetLastError();
}

template <int M, int EPI, int PRE>
static hipError_t gemv_lpr(const bf16_t* W, const bf16_t* X, int ldx, int N, int K, float eps,
                           const EpiArgs& ea, hipStream_t st) {
  if (K <= 1024) return launch_gemv<M, 32, EPI, PRE>(W, X, ldx, N, K, eps, ea, st);
  return launch_gemv<M, 64, EPI, PRE>(W, X, ldx, N, K, eps, ea, st);
}

template <int M>
static hipError_t gemv_m(int epi, int pre, const bf16_t* W, const bf16_t* X, int ldx, int N,
                         int K, float eps, const EpiArgs& ea, hipStream_t st) {
#define ANN_GEMV_PRE(E)                                                                 \
  switch (pre) {                                                                        \
    case PRE_PLAIN: return gemv_lpr<M, E, PRE_PLAIN>(W, X, ldx, N, K, eps, ea, st); \
    case PRE_RMS: return gemv_lpr<M, E, PRE_RMS>(W, X, ldx, N, K, eps, ea, st);     \
  }                                                                                     \
  break;
  switch (epi) {
    case EPI_STORE: ANN_GEMV_PRE(EPI_STORE)
    case EPI_RELU2: ANN_GEMV_PRE(EPI_RELU2)
    case EPI_RESID_ATTN: ANN_GEMV_PRE(EPI_RESID_ATTN)
    case EPI_RESID_MLP: ANN_GEMV_PRE(EPI_RESID_MLP)
    case EPI_LOGITS: ANN_GEMV_PRE(EPI_LOGITS)
  }
#undef ANN_GEMV_PRE
  return hipErrorInvalidValue;
}

hipError_t gemv(int epi, int pre, const bf16_t* W, const bf16_t* X, int ldx, int M, int N, int K,
                float eps, const EpiArgs& ea, hipStream_t st) {
  if (!gemv_fits(M, K)) return hipErrorInvalidValue;
  switch (M) {
    case 1: return gemv_m<1>(epi, pre, W, X, ldx, N, K, eps, ea, st);
    case 2: return gemv_m<2>(epi, pre, W, X, ldx, N, K, eps, ea, st);
    case 3: return gemv_m<3>(epi, pre, W, X, ldx, N, K, eps, ea, st);
    case 4: return gemv_m<4>(epi, pre, W, X, ldx, N, K, eps, ea, st);
    case 5: return gemv_m<5>(epi, pre, W, X, ldx, N, K, eps, ea, st);
    case 6: return gemv_m<6>(epi, pre, W, X, ldx, N, K, eps, ea, st);
    case 7: return gemv_m<7>(epi, pre, W, X, ldx, N, K, eps, ea, st);
    case 8: return gemv_m<8>(epi, pre, W, X, ldx, N, K, eps, ea, st);
  }
  return hipErrorInvalidValue;
}

// ---- lm_head top-k candidates (EPI_TOPK) ------------------------------------

// max of v over the 16 lanes of each DPP row (lanes 16r .. 16r + 15): quad
// swaps 1 and 2, then the half-row and row mirrors
__device__ __forceinline__ uint32_t row16_max(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
  return v;
}

// descending compare-exchange
__device__ __forceinline__ void cas_desc(uint32_t& a, uint32_t& b) {
  const uint32_t hi = max(a, b), lo = min(a, b);
  a = hi;
  b = lo;
}

// Candidates of a staged bf16 tile (BM x 128, row pitch CP) of lm_head
// outputs at (m0, n0), column tile tn.  A 16-lane row of the wave takes one
// output row, 8 columns per lane, RP rows at a time (independent chains).
// Each lane sorts its words (zkey << 16 | 0xffff - n; distinct, as the
// columns are) in descending order; nine rounds of a row maximum over the
// lanes' first words then pop the largest word from its lane: rounds 0-7 are
// the candidates, largest first, round 8 the 9th largest word (0 when fewer
// valid columns remain).  The fp32 softcapped logits are stored from the
// same tile when requested.
template <int BM, int CP>
__device__ __forceinline__ void topk_tile_epilogue(const EpiArgs& ea, const bf16_t* tile, int m0,
                                                   int n0, int M, int N, int tn, int tid) {
  constexpr int RP = 4;
  static_assert(BM % (16 * RP) == 0, "whole row groups");
  const int grp = tid >> 4, li = tid & 15;
  const int nb = n0 + li * 8;
#pragma unroll 1
  for (int p = 0; p < BM / 16; p += RP) {
    uint32_t w[RP][8];
#pragma unroll
    for (int q = 0; q < RP; ++q) {
      const int ml = (p + q) * 16 + grp, m = m0 + ml;
      const uint4 v = *(const uint4*)(tile + ml * CP + li * 8);
      const uint32_t hw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const bf16_t h = (bf16_t)(e & 1 ? hw[e >> 1] >> 16 : hw[e >> 1] & 0xffffu);
        w[q][e] = nb + e < ea.Vs ? (zkey(h) << 16) | (0xffffu - (uint32_t)(nb + e)) : 0u;
      }
      if (ea.logits && m < M) {
        float* lr = ea.logits + (size_t)m * ea.ldz + nb;
        if (nb + 7 < N && (ea.ldz & 3) == 0) {
          float f[8];
#pragma unroll
          for (int e = 0; e < 8; ++e)
            f[e] = softcap(__uint_as_float(e & 1 ? hw[e >> 1] & 0xffff0000u : hw[e >> 1] << 16));
          *(float4*)lr = make_float4(f[0], f[1], f[2], f[3]);
          *(float4*)(lr + 4) = make_float4(f[4], f[5], f[6], f[7]);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (nb + e < N)
              lr[e] = softcap(__uint_as_float(e & 1 ? hw[e >> 1] & 0xffff0000u : hw[e >> 1] << 16));
        }
      }
      if (ea.tk_first) continue;   // greedy: the maximum only (below)
      // Batcher's odd-even merge sort of 8, descending
      uint32_t(&x)[8] = w[q];
      cas_desc(x[0], x[1]); cas_desc(x[2], x[3]); cas_desc(x[4], x[5]); cas_desc(x[6], x[7]);
      cas_desc(x[0], x[2]); cas_desc(x[1], x[3]); cas_desc(x[4], x[6]); cas_desc(x[5], x[7]);
      cas_desc(x[1], x[2]); cas_desc(x[5], x[6]);
      cas_desc(x[0], x[4]); cas_desc(x[1], x[5]); cas_desc(x[2], x[6]); cas_desc(x[3], x[7]);
      cas_desc(x[2], x[4]); cas_desc(x[3], x[5]);
      cas_desc(x[1], x[2]); cas_desc(x[3], x[4]); cas_desc(x[5], x[6]);
    }
    if (ea.tk_first) {   // greedy rows: each tile's largest word
#pragma unroll
      for (int q = 0; q < RP; ++q) {
        uint32_t lm = w[q][0];
#pragma unroll
        for (int e = 1; e < 8; ++e) lm = max(lm, w[q][e]);
        const uint32_t g = row16_max(lm);
        const int m = m0 + (p + q) * 16 + grp;
        if (m < M && li == 0) ea.cand[((size_t)m * ea.nt + tn) * TK_M] = g;
      }
      continue;
    }
    uint32_t mine[RP];   // lane li < 8: candidate li; lane 8: the 9th word
#pragma unroll
    for (int q = 0; q < RP; ++q) mine[q] = 0u;
#pragma unroll
    for (int r = 0; r <= TK_M; ++r) {
#pragma unroll
      for (int q = 0; q < RP; ++q) {
        const uint32_t g = row16_max(w[q][0]);
        if (li == r) mine[q] = g;
        if (r < TK_M && w[q][0] == g) {
#pragma unroll
          for (int e = 0; e < 7; ++e) w[q][e] = w[q][e + 1];
          w[q][7] = 0u;
        }
      }
    }
#pragma unroll
    for (int q = 0; q < RP; ++q) {
      const int m = m0 + (p + q) * 16 + grp;
      if (m < M) {
        const size_t rec = (size_t)m * ea.nt + tn;
        if (li < TK_M) ea.cand[rec * TK_M + li] = mine[q];
        else if (li == TK_M) ea.cand_r[rec] = mine[q];
      }
    }
  }
}

// ---- MFMA GEMM, large M (prefill) -------------------------------------------
//
// 128 x 128 x 64 block tiles, 4 waves of 64 x 64 (4 x 4 blocks of
// v_mfma_f32_16x16x32_bf16), K tiles staged through XOR-swizzled LDS with the
// next tile prefetched into registers during the MFMAs.  A arrives already
// normalised (rms_apply) when the projection needs it.

constexpr int GM_BM = 128, GM_BN = 128, GM_BK = 64;

// LDS layout of a K tile: unpadded 128-byte rows, the 16-byte chunk c of row
// r at slot c ^ ((r >> 1) & 7).  The LDS serves 16 lanes of a 16-byte access
// per cycle over 64 banks (256 B): the MFMA fragment reads (16 rows, one
// chunk) and the tile stores (2 rows, 8 chunks) both hit 16 distinct 16-byte
// bank groups.  The padded layout (+16 B per row) left the stores 2-way
// conflicted; measured 5-10% faster on the prefill shapes.
__device__ __forceinline__ int gm_lds(int row, int c) {
  return row * GM_BK + ((c ^ ((row >> 1) & 7)) << 3);
}

// Work-group tile BM x BN, four waves of BM/2 x BN/2.  BM = 64 when M <= 64
// (no padding rows in the MFMAs: the batch-64 lm_head runs 1.4x faster
// measured), 128 below 512 rows, 256 x 128 / 128 x 256 above (k_gemm_2w).
// DEPTH: K tiles in flight per thread (a register ring; 1 = the next tile
// only).  Each K tile of a thread is one memory round trip after the tile
// before it is stored: with few work-groups and short K loops (decode) a
// deeper ring keeps more bytes in flight per CU.
template <int EPI, int BM, int BN, int DEPTH = 1>
__device__ __forceinline__ void gemm_body(const bf16_t* __restrict__ A, int lda,
                                          const bf16_t* __restrict__ W, int M, int N, int K,
                                          const EpiArgs& ea) {
  constexpr int AC = BM * GM_BK / 8 / 256;   // 16-byte A chunks per thread per K tile
  constexpr int BC = BN * GM_BK / 8 / 256;   // and of W
  constexpr int WM = BM / 2, MT = WM / 16;   // rows per wave, 16-row MFMA tiles per wave
  constexpr int WN = BN / 2, NT = WN / 16;   // columns per wave, 16-column tiles per wave
  constexpr int CH = AC > BC ? AC : BC;
  // the QKV and CE epilogues work on 128-column tiles (whole heads; the
  // per-tile partial sums of the loss)
  static_assert((EPI != EPI_QKV && EPI != EPI_CE) || BN == GM_BN, "128-column tiles");
  static_assert(EPI != EPI_TOPK || BN % 128 == 0, "whole 128-column candidate tiles");
  // staged epilogues (QKV; PE_B / PE_X on full tiles) reuse the LDS for a bf16
  // BM x BN tile of row pitch BN + 8
  // the batched plain store stages its 128 x 128 tiles for the symmetric form
  constexpr bool STAGE_STORE = EPI == EPI_STORE && BM == GM_BM && BN == GM_BN && DEPTH == 1;
  constexpr bool STAGED =
      EPI == EPI_QKV || EPI == EPI_PE_B || EPI == EPI_PE_X || EPI == EPI_TOPK || STAGE_STORE;
  constexpr int SMEM = (BM + BN) * GM_BK > (STAGED ? BM * (BN + 8) : 0)
                           ? (BM + BN) * GM_BK
                           : BM * (BN + 8);
  __shared__ __attribute__((aligned(16))) bf16_t smem[SMEM];
  bf16_t* As = smem;
  bf16_t* Bs = smem + BM * GM_BK;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv >> 1, wn = wv & 1;
  // XCD-aware tile order: work-groups are dispatched round-robin over the 8
  // XCDs, so work-group b runs on XCD b % 8.  Each XCD takes a contiguous
  // range of tiles in (M block, N block) row-major order: the N tiles of one
  // M block then share their A rows in that XCD's L2.  A bijection of the
  // grid (correct under any dispatch order); batched launches keep the
  // identity.  Measured 3-6% faster per prefill GEMM.
  int tm = blockIdx.y, tn = blockIdx.x;
  if (ea.sym) {
    // symmetric output: blockIdx.x walks the tiles tn >= tm row by row
    const int nb = (M + BM - 1) / BM;
    int t = blockIdx.x;
    tm = 0;
    while (t >= nb - tm) {
      t -= nb - tm;
      ++tm;
    }
    tn = tm + t;
  } else if (gridDim.z == 1) {
    const int nbn = gridDim.x, total = nbn * gridDim.y;
    const int bid = blockIdx.y * nbn + blockIdx.x;
    const int x = bid & 7, q = total >> 3, r = total & 7;
    const int t = x * q + min(x, r) + (bid >> 3);
    tm = t / nbn;
    tn = t - tm * nbn;
  }
  const int m0 = tm * BM, n0 = tn * BN;

  // each thread moves AC 16-byte chunks of A and BC of W per K tile
  int arow[CH], acol[CH];
  bool aok[CH], bok[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int id = tid + i * 256;
    arow[i] = id >> 3;
    acol[i] = (id & 7) * 8;
    aok[i] = i < AC && (m0 + arow[i]) < M;
    bok[i] = i < BC && (n0 + arow[i]) < N;
  }
  u32x4_t ra[DEPTH][AC], rb[DEPTH][BC];
  // DEPTH > 1: rows past M / N load the last valid row instead (they feed
  // only outputs that are never stored), so every load is unconditional and
  // the compiler can wait on the oldest slot alone (vmcnt(N)) instead of on
  // every load in flight
  const bf16_t* pa[AC];
  const bf16_t* pb[BC];
#pragma unroll
  for (int i = 0; i < AC; ++i)
    pa[i] = A + (size_t)min(m0 + arow[i], M - 1) * lda + acol[i];
#pragma unroll
  for (int i = 0; i < BC; ++i) pb[i] = W + (size_t)min(n0 + arow[i], N - 1) * K + acol[i];
  auto load_tile = [&](auto slc, int k0) __attribute__((always_inline)) {
    constexpr int sl = decltype(slc)::value;
    if constexpr (DEPTH > 1) {
#pragma unroll
      for (int i = 0; i < AC; ++i) ra[sl][i] = *(const u32x4_t*)(pa[i] + k0);
#pragma unroll
      for (int i = 0; i < BC; ++i) rb[sl][i] = *(const u32x4_t*)(pb[i] + k0);
      return;
    }
#pragma unroll
    for (int i = 0; i < AC; ++i)
      ra[sl][i] = aok[i] ? *(const u32x4_t*)(A + (size_t)(m0 + arow[i]) * lda + k0 + acol[i])
                         : (u32x4_t){0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < BC; ++i)
      rb[sl][i] = bok[i] ? *(const u32x4_t*)(W + (size_t)(n0 + arow[i]) * K + k0 + acol[i])
                         : (u32x4_t){0u, 0u, 0u, 0u};
  };
  auto store_tile = [&](auto slc) __attribute__((always_inline)) {
    constexpr int sl = decltype(slc)::value;
#pragma unroll
    for (int i = 0; i < AC; ++i) *(u32x4_t*)(As + gm_lds(arow[i], acol[i] >> 3)) = ra[sl][i];
#pragma unroll
    for (int i = 0; i < BC; ++i) *(u32x4_t*)(Bs + gm_lds(arow[i], acol[i] >> 3)) = rb[sl][i];
  };

  // SWAP: acc[j][i] is block (N block j, M block i) of C^T = W A^T, so that a
  // lane holds four consecutive columns n of one row m (8-byte epilogue
  // accesses); otherwise block (M block i, N block j) of C = A W^T, a lane
  // holding one column of four rows.  Measured: the read-modify-write
  // epilogues gain from SWAP (prefill o / proj 20 us each), the plain stores
  // lose (qkv / fc 16 us each).
  constexpr bool SWAP = EPI != EPI_STORE && EPI != EPI_RELU2;
  floatx4_t acc[NT][MT];
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[j][i] = (floatx4_t){0.f, 0.f, 0.f, 0.f};

  // fragment rows are 16-row aligned + r16: slot of chunk c is c ^ ((r16 >> 1) & 7)
  const int r16 = lane & 15, kg = lane >> 4, sw = (r16 >> 1) & 7;
  // DEPTH > 1 needs K / GM_BK a multiple of DEPTH (host-checked): no break
  // and no conditional load in the loop; the last DEPTH refills re-read the
  // last tile (unused)
  const int KT = K / GM_BK;
  static_for<0, DEPTH>([&](auto slc) __attribute__((always_inline)) {
    load_tile(slc, decltype(slc)::value * GM_BK);
  });
  for (int kt0 = 0; kt0 < KT; kt0 += DEPTH)
  static_for<0, DEPTH>([&](auto slc) __attribute__((always_inline)) {
    const int kt = kt0 + decltype(slc)::value;
    __syncthreads();
    store_tile(slc);
    __syncthreads();
    if constexpr (DEPTH > 1)
      load_tile(slc, min(kt + DEPTH, KT - 1) * GM_BK);
    else if (kt + 1 < KT)
      load_tile(slc, (kt + 1) * GM_BK);
#pragma unroll
    for (int kk = 0; kk < GM_BK; kk += 32) {
      bf16x8_t a[MT], b[NT];
#pragma unroll
      for (int i = 0; i < MT; ++i)
        a[i] = *(const bf16x8_t*)(As + (wm * WM + i * 16 + r16) * GM_BK +
                                  ((((kk >> 3) + kg) ^ sw) << 3));
#pragma unroll
      for (int j = 0; j < NT; ++j)
        b[j] = *(const bf16x8_t*)(Bs + (wn * WN + j * 16 + r16) * GM_BK +
                                  ((((kk >> 3) + kg) ^ sw) << 3));
      if constexpr (SWAP) {
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int i = 0; i < MT; ++i)
            acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b[j], a[i], acc[j][i], 0, 0, 0);
      } else {
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int j = 0; j < NT; ++j)
            acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[j][i], 0, 0, 0);
      }
    }
  });
  // tile^T of the staged bf16 tile (row pitch CP) to dst[(n0 + c) * ld + m0 + r]:
  // a thread takes a column pair and a band of rows, 16-byte runs
  auto store_transposed = [&](bf16_t* dst, int ld, auto cpc) __attribute__((always_inline)) {
    constexpr int CP = decltype(cpc)::value;
    constexpr int NP = BN / 2, TB = 256 / NP, RB = BM / TB;
    const int cp = tid % NP, rb = tid / NP;
#pragma unroll
    for (int g = 0; g < RB / 8; ++g) {
      const int r0 = rb * RB + 8 * g;
      uint32_t w[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) w[e] = *(const uint32_t*)(smem + (r0 + e) * CP + 2 * cp);
      uint4 c0, c1;
      c0.x = (w[0] & 0xffffu) | (w[1] << 16); c0.y = (w[2] & 0xffffu) | (w[3] << 16);
      c0.z = (w[4] & 0xffffu) | (w[5] << 16); c0.w = (w[6] & 0xffffu) | (w[7] << 16);
      c1.x = (w[0] >> 16) | (w[1] & 0xffff0000u); c1.y = (w[2] >> 16) | (w[3] & 0xffff0000u);
      c1.z = (w[4] >> 16) | (w[5] & 0xffff0000u); c1.w = (w[6] >> 16) | (w[7] & 0xffff0000u);
      bf16_t* t0 = dst + (size_t)(n0 + 2 * cp) * ld + m0 + r0;
      *(uint4*)t0 = c0;
      *(uint4*)(t0 + ld) = c1;
    }
  };
  if constexpr (!SWAP) {
    // C layout of the 16x16 MFMA: lane holds column (lane & 15), rows 4 (lane >> 4) + r
    if constexpr (STAGE_STORE) {
      // symmetric form (full tiles, host-checked): staged bf16 tile, 16-byte
      // row chunks, and the mirrored tile^T above the diagonal
      if (ea.sym) {
        constexpr int CP = BN + 8, CPR = BN / 8, NCH = BM * CPR / 256;
        __syncthreads();   // every wave is done with the last K tile in LDS
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              smem[(wm * WM + i * 16 + (lane >> 4) * 4 + r) * CP + wn * WN + j * 16 + r16] =
                  f2bf(acc[j][i][r]);
        __syncthreads();
#pragma unroll
        for (int u = 0; u < NCH; ++u) {
          const int q = tid + 256 * u, ml = q / CPR, c8 = (q % CPR) * 8;
          *(uint4*)(ea.out + (size_t)(m0 + ml) * ea.ldo + n0 + c8) =
              *(const uint4*)(smem + ml * CP + c8);
        }
        if (tn != tm) store_transposed(ea.out, ea.ldo, std::integral_constant<int, CP>{});
        return;
      }
    }
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int n = n0 + wn * WN + j * 16 + r16;
        if (n >= N) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + wm * WM + i * 16 + (lane >> 4) * 4 + r;
          if (m < M) epilogue<EPI>(ea, m, n, acc[j][i][r]);
        }
      }
    return;
  }
  // C^T layout: lane holds column m = (lane & 15) of its M block and rows
  // n = 4 (lane >> 4) + r, r = 0..3, of its N block
  if constexpr (EPI == EPI_CE) {
    // softcap(bf16(z)) in (0, 23): sum exp(zc) needs no max pass.  Row sums:
    // in-lane over the wave's 4 N blocks, then over the 4 lane groups, then
    // the two column halves (wn) through LDS, always in the same order.  The
    // softcap and exp use the hardware exp2 / reciprocal: the IEEE expf and
    // division cost ~35 VALU instructions per logit, over 1.65 G logits in the
    // 64 x 512-token forward
    float rs[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int m = m0 + wm * WM + i * 16 + r16;
      const int tg = m < M ? ea.tgt[m] : -1;
      float sum = 0.f;
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int n = n0 + wn * WN + j * 16 + (lane >> 4) * 4 + r;
          if (n < N) {
            const float zc = softcap_fast(bf2f(f2bf(acc[j][i][r])));
            sum += __builtin_amdgcn_exp2f(zc * 1.4426950408889634f);
            if (n == tg) ea.ce_tz[m] = zc;
          }
        }
      sum += __shfl_xor(sum, 16, 64);
      sum += __shfl_xor(sum, 32, 64);
      rs[i] = sum;
    }
    __syncthreads();   // LDS tiles no longer read: reuse for the halves
    float* red = (float*)smem;
    if (wn == 1 && lane < 16) {
#pragma unroll
      for (int i = 0; i < MT; ++i) red[wm * WM + i * 16 + r16] = rs[i];
    }
    __syncthreads();
    if (wn == 0 && lane < 16) {
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int m = m0 + wm * WM + i * 16 + r16;
        if (m < M) ea.ce_part[(size_t)tn * ea.ldz + m] = rs[i] + red[wm * WM + i * 16 + r16];
      }
    }
  } else if constexpr (EPI == EPI_QKV) {
    QkvRows<BM> pr;
    qkv_prefetch<BM>(ea, m0, M, tid, pr);
    __syncthreads();   // every wave is done with the last K tile in LDS
    constexpr int CP = BN + 8;
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const floatx4_t y = acc[j][i];
        *(uint2*)(smem + (wm * WM + i * 16 + r16) * CP + wn * WN + j * 16 + (lane >> 4) * 4) =
            make_uint2(pack2(y[0], y[1]), pack2(y[2], y[3]));
      }
    __syncthreads();
    qkv_tile_epilogue<BM, GM_BN + 8>(ea, smem, m0, n0, M, tid, pr);
  } else if constexpr (EPI == EPI_TOPK) {
    __syncthreads();   // every wave is done with the last K tile in LDS
    constexpr int CP = BN + 8;
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const floatx4_t y = acc[j][i];
        *(uint2*)(smem + (wm * WM + i * 16 + r16) * CP + wn * WN + j * 16 + (lane >> 4) * 4) =
            make_uint2(pack2(y[0], y[1]), pack2(y[2], y[3]));
      }
    __syncthreads();
#pragma unroll
    for (int hf = 0; hf < BN / 128; ++hf)
      if (tn * (BN / 128) + hf < ea.nt)
        topk_tile_epilogue<BM, CP>(ea, smem + hf * 128, m0, n0 + hf * 128, M, N,
                                   tn * (BN / 128) + hf, tid);
  } else {
    if constexpr (EPI == EPI_PE_B || EPI == EPI_PE_X) {
      // full tiles with 16-byte rows: x prefetched before the staging
      // barrier, bf16(y) staged in LDS (exact: both epilogues start from
      // bf16(y)), 16-byte row chunks mixed and stored, and for PE_X the
      // transposed copy written from LDS as 16-byte column runs.  Measured
      // against per-lane 8-byte accesses and 2-byte transposed stores.
      const bool full = m0 + BM <= M && n0 + BN <= N && ((ea.ldr | ea.ldo) & 7) == 0 &&
                        (((uintptr_t)ea.x | (uintptr_t)ea.out) & 15) == 0 &&
                        (EPI != EPI_PE_X || !ea.outT ||
                         ((ea.ldoT & 7) == 0 && ((uintptr_t)ea.outT & 15) == 0));
      if (full) {
        constexpr int CP = BN + 8, CPR = BN / 8, NCH = BM * CPR / 256;
        static_assert(BM * CPR % 256 == 0, "whole chunks per thread");
        uint4 xv[NCH];
#pragma unroll
        for (int u = 0; u < NCH; ++u) {
          const int q = tid + 256 * u;
          xv[u] = *(const uint4*)(ea.x + (size_t)(m0 + q / CPR) * ea.ldr + n0 + (q % CPR) * 8);
        }
        __syncthreads();   // every wave is done with the last K tile in LDS
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int i = 0; i < MT; ++i) {
            const floatx4_t y = acc[j][i];
            *(uint2*)(smem + (wm * WM + i * 16 + r16) * CP + wn * WN + j * 16 + (lane >> 4) * 4) =
                make_uint2(pack2(y[0], y[1]), pack2(y[2], y[3]));
          }
        __syncthreads();
        const float s0 = ea.s0, s1 = ea.s1;
#pragma unroll
        for (int u = 0; u < NCH; ++u) {
          const int q = tid + 256 * u, ml = q / CPR, c8 = (q % CPR) * 8;
          uint4* sy = (uint4*)(smem + ml * CP + c8);
          const uint4 yv = *sy;
          const uint32_t xw[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
          const uint32_t yw[4] = {yv.x, yv.y, yv.z, yv.w};
          uint32_t o[4];
#pragma unroll
          for (int f = 0; f < 4; ++f) {
            const uint32_t a = pack2(s0 * lo_f(xw[f]), s0 * hi_f(xw[f]));
            uint32_t b = yw[f];
            if constexpr (EPI == EPI_PE_B) b = pack2(s1 * lo_f(b), s1 * hi_f(b));
            o[f] = pack2(lo_f(a) + lo_f(b), hi_f(a) + hi_f(b));
          }
          const uint4 ov = make_uint4(o[0], o[1], o[2], o[3]);
          *(uint4*)(ea.out + (size_t)(m0 + ml) * ea.ldo + n0 + c8) = ov;
          *sy = ov;   // kept for a transposed copy
        }
        // PE_X: the transposed copy x'^T; PE_B in the symmetric form: the
        // mirrored tile above the diagonal
        bf16_t* tdst = nullptr;
        int tld = 0;
        if constexpr (EPI == EPI_PE_X) {
          tdst = ea.outT;
          tld = ea.ldoT;
        } else if (ea.sym && tn != tm) {
          tdst = ea.out;
          tld = ea.ldo;
        }
        if (tdst) {
          __syncthreads();
          store_transposed(tdst, tld, std::integral_constant<int, CP>{});
        }
        return;
      }
    }
    const bool vec = epi_vec_ok<EPI>(ea);
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int n = n0 + wn * WN + j * 16 + (lane >> 4) * 4;
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int m = m0 + wm * WM + i * 16 + r16;
        if (m < M) epilogue4<EPI>(ea, vec, m, n, N, acc[j][i]);
      }
    }
  }
}

template <int EPI, int BM, int BN>
__global__ __launch_bounds__(256) void k_gemm(const bf16_t* __restrict__ A, int lda,
                                              const bf16_t* __restrict__ W, int M, int N, int K,
                                              EpiArgs ea) {
  gemm_body<EPI, BM, BN>(A, lda, W, M, N, K, ea);
}

// Decode projections of 65-128 rows (64 x 64 tiles, about 200 work-groups):
// DEPTH K tiles in flight per thread.
template <int EPI, int BM, int BN, int DEPTH>
__global__ __launch_bounds__(256) void k_gemm_deep(const bf16_t* __restrict__ A, int lda,
                                                   const bf16_t* __restrict__ W, int M, int N,
                                                   int K, EpiArgs ea) {
  gemm_body<EPI, BM, BN, DEPTH>(A, lda, W, M, N, K, ea);
}

// The 256 x 128 and 128 x 256 tiles (waves of 128 x 64 / 64 x 128: a quarter
// less LDS traffic per flop than 64 x 64) held to two waves per SIMD, so two
// work-groups share a CU.  Measured 10-15% faster than 128 x 128 on the
// prefill shapes; without the register cap the compiler takes one wave per
// SIMD and they are slower.
template <int EPI, int BM, int BN>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_gemm_2w(
    const bf16_t* __restrict__ A, int lda, const bf16_t* __restrict__ W, int M, int N, int K,
    EpiArgs ea) {
  gemm_body<EPI, BM, BN>(A, lda, W, M, N, K, ea);
}

// Batched: blockIdx.z selects matrix z; A, W, the output and the epilogue's
// second operand (x) advance by their batch strides.
template <int EPI, int BM>
__global__ __launch_bounds__(256) void k_gemm_bat(const bf16_t* __restrict__ A, int lda,
                                                  long long sA, const bf16_t* __restrict__ W,
                                                  long long sW, int M, int N, int K, EpiArgs ea,
                                                  long long sOut, long long sX) {
  const long long z = blockIdx.z;
  ea.out += z * sOut;
  ea.x += z * sX;
  if (ea.outT) ea.outT += z * sOut;   // same shape as out
  gemm_body<EPI, BM, GM_BN>(A + z * sA, lda, W + z * sW, M, N, K, ea);
}

// ---- skinny MFMA GEMM (decode, M <= 128): the body is in sk_gemm.h -----------

template <int EPI, bool RMS, int KB, int T>
__global__ __launch_bounds__(256) void k_gemm_sk(const bf16_t* __restrict__ A, int lda,
                                                 const bf16_t* __restrict__ W, int M, int N, int K,
                                                 float eps, EpiArgs ea) {
  gemm_sk_body<RMS, KB, T>(A, lda, W, M, N, K, eps, blockIdx.x, blockIdx.y,
                           [&](int m, int n, const floatx4_t& v) {
#pragma unroll
                             for (int r = 0; r < 4; ++r)
                               if (m + r < M && n < N) epilogue<EPI>(ea, m + r, n, v[r]);
                           });
}

// ---- skinny MFMA GEMM, LDS-staged (decode, M <= 128, no RMS prologue) ------
//
// Same work split as k_gemm_sk (one 16T x 16T tile per work-group, the four
// waves split K into quarters), but each wave brings its quarter of the A and
// W tiles in with contiguous 16-byte loads -- lanes along a row, not the
// 16-row x 64-byte MFMA fragment pattern, which moves ~3x fewer bytes per CU
// cycle -- into its own padded LDS region, in rounds of KC k-steps, and reads
// the fragments back with ds_read_b128.  A wave touches only its own region,
// so no barrier is needed until the cross-wave sum, whose partials go into
// each wave's own (then finished) region.  Operands are swapped for the
// read-modify-write epilogues (8-byte accesses), as in k_gemm.  Bit-identical
// to k_gemm_sk (same k order per wave, same wave order).
// RMS: the rows of A are normalised in the kernel (model.py:48-49 with the
// bf16 output of an eager op): before the first round each wave reads its K
// quarter of the tile's A rows with contiguous loads, leaves per-chunk sums of
// squares in its own (not yet used) LDS region, sums each row's chunks in
// order and the quarters are added in wave order; the fragments are then
// scaled and rounded to bf16 as they come out of LDS.
// D: rounds in flight per wave (a register ring): round r + D is loaded as
// soon as round r is in LDS, so a wave waits on memory about once per D
// rounds instead of once per round.
template <int EPI, bool RMS, int KC, int T, int D>
__global__ __launch_bounds__(256) void k_gemm_sk2(const bf16_t* __restrict__ A, int lda,
                                                  const bf16_t* __restrict__ W, int M, int N,
                                                  int K, float eps, EpiArgs ea) {
  constexpr int R = 16 * T;        // rows per operand tile
  constexpr int CPR = 4 * KC;      // 16-byte chunks per row per round
  constexpr int PITCH = CPR + 1;   // padded row pitch, in uint4
  constexpr int NL = R * CPR / 64; // loads per lane per operand per round
  constexpr int REGION = 2 * R * PITCH;
  static_assert(REGION * 16 >= T * T * 64 * 16, "partials fit a wave's region");
  constexpr bool SWAP = EPI != EPI_STORE && EPI != EPI_RELU2;
  __shared__ uint4 s_t[4][REGION];
  __shared__ float s_ss[RMS ? 4 : 1][R];
  const int tid = threadIdx.x, lane = tid & 63, wk = tid >> 6;
  const int n0 = blockIdx.x * 16 * T, m0 = blockIdx.y * 16 * T;
  const int kw = K >> 7;            // k-steps of 32 per wave
  const int kbase = wk * kw * 32;   // first k of this wave's quarter
  uint4* sa = s_t[wk];
  uint4* sw = s_t[wk] + R * PITCH;
  floatx4_t acc[T][T];
#pragma unroll
  for (int i = 0; i < T; ++i)
#pragma unroll
    for (int j = 0; j < T; ++j) acc[i][j] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  const int r16 = lane & 15, q4 = lane >> 4;
  float scale[T];
#pragma unroll
  for (int t = 0; t < T; ++t) scale[t] = 1.f;
  if (RMS) {   // host guarantees R * 4 kw floats fit the region
    const int cq = 4 * kw;          // chunks of a row in this quarter
    float* ps = (float*)s_t[wk];
    for (int c0 = 0; c0 < R * cq; c0 += 8 * 64) {   // eight loads in flight per lane
      uint4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int c = c0 + 64 * u + lane;
        const int row = c / cq, col = c % cq;
        v[u] = (c < R * cq && m0 + row < M)
                   ? *(const uint4*)(A + (size_t)(m0 + row) * lda + kbase + col * 8)
                   : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int c = c0 + 64 * u + lane;
        float f[8];
        unpack8(v[u], f);
        float q = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) q += f[j] * f[j];
        if (c < R * cq) ps[c] = q;
      }
    }
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
    if (lane < R) {
      float q = 0.f;
      for (int col = 0; col < cq; ++col) q += ps[lane * cq + col];
      s_ss[wk][lane] = q;
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int r = 16 * t + r16;
      const float tt = ((s_ss[0][r] + s_ss[1][r]) + s_ss[2][r]) + s_ss[3][r];
      scale[t] = rsqrtf(tt / (float)K + eps);
    }
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
  }
  u32x4_t ca[D][NL], cw[D][NL];
  auto load_round = [&](auto slc, int s0) __attribute__((always_inline)) {
    constexpr int sl = decltype(slc)::value;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int c = 64 * i + lane;
      const int row = c / CPR, col = c % CPR;
      if constexpr (D > 1) {
        // unconditional loads (clamped rows / k-steps feed only outputs and
        // k-steps that are never used), so the compiler waits on the oldest
        // round alone instead of on every load in flight
        const int am = min(m0 + row, M - 1), wn = min(n0 + row, N - 1);
        const size_t ke = (size_t)kbase + (size_t)min(s0 + col / 4, kw - 1) * 32 + (col & 3) * 8;
        ca[sl][i] = *(const u32x4_t*)(A + (size_t)am * lda + ke);
        cw[sl][i] = *(const u32x4_t*)(W + (size_t)wn * K + ke);
      } else {
        const bool ok = s0 + col / 4 < kw;
        const int am = m0 + row, wn = n0 + row;
        const size_t ke = (size_t)kbase + (size_t)s0 * 32 + col * 8;
        ca[sl][i] = (ok && am < M) ? *(const u32x4_t*)(A + (size_t)am * lda + ke)
                                   : (u32x4_t){0u, 0u, 0u, 0u};
        cw[sl][i] = (ok && wn < N) ? *(const u32x4_t*)(W + (size_t)wn * K + ke)
                                   : (u32x4_t){0u, 0u, 0u, 0u};
      }
    }
  };
  // D > 1 needs the round count a multiple of D (host-checked): no break and
  // no conditional load in the loop; the last D refills re-read the last round
  const int nrounds = (kw + KC - 1) / KC;
  static_for<0, D>([&](auto slc) __attribute__((always_inline)) {
    load_round(slc, decltype(slc)::value * KC);
  });
  for (int r0 = 0; r0 < nrounds; r0 += D)
  static_for<0, D>([&](auto slc) __attribute__((always_inline)) {
    constexpr int sl = decltype(slc)::value;
    const int rd = r0 + sl;
    const int s0 = rd * KC;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int c = 64 * i + lane;
      const int row = c / CPR, col = c % CPR;
      *(u32x4_t*)&sa[row * PITCH + col] = ca[sl][i];
      *(u32x4_t*)&sw[row * PITCH + col] = cw[sl][i];
    }
    // LDS accesses of one wave complete in order: its reads below see its
    // writes above; this keeps the compiler from reordering them
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
    if constexpr (D > 1)
      load_round(slc, min(rd + D, nrounds - 1) * KC);
    else if (rd + 1 < nrounds)
      load_round(slc, (rd + 1) * KC);
#pragma unroll
    for (int s = 0; s < KC; ++s) {
      if (D > 1 || s0 + s < kw) {   // D > 1: whole rounds (host-checked)
        uint4 a[T], w[T];
#pragma unroll
        for (int t = 0; t < T; ++t) {
          a[t] = sa[(16 * t + r16) * PITCH + 4 * s + q4];
          w[t] = sw[(16 * t + r16) * PITCH + 4 * s + q4];
          if (RMS) {
            float f[8];
            unpack8(a[t], f);
            a[t] = make_uint4(pack2(f[0] * scale[t], f[1] * scale[t]),
                              pack2(f[2] * scale[t], f[3] * scale[t]),
                              pack2(f[4] * scale[t], f[5] * scale[t]),
                              pack2(f[6] * scale[t], f[7] * scale[t]));
          }
        }
#pragma unroll
        for (int ta = 0; ta < T; ++ta)
#pragma unroll
          for (int tw = 0; tw < T; ++tw)
            acc[ta][tw] = SWAP ? __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                     *(bf16x8_t*)&w[tw], *(bf16x8_t*)&a[ta], acc[ta][tw], 0, 0, 0)
                               : __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                     *(bf16x8_t*)&a[ta], *(bf16x8_t*)&w[tw], acc[ta][tw], 0, 0, 0);
      }
    }
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
  });
  // partials of waves 1..3 into their own regions, summed by wave 0 in order
  floatx4_t* red = (floatx4_t*)s_t[wk];
  if (wk > 0) {
#pragma unroll
    for (int ta = 0; ta < T; ++ta)
#pragma unroll
      for (int tw = 0; tw < T; ++tw) red[(ta * T + tw) * 64 + lane] = acc[ta][tw];
  }
  __syncthreads();
  if (wk > 0) return;
  const bool vec = SWAP && epi_vec_ok<EPI>(ea);
#pragma unroll
  for (int ta = 0; ta < T; ++ta)
#pragma unroll
    for (int tw = 0; tw < T; ++tw) {
      floatx4_t v = acc[ta][tw];
#pragma unroll
      for (int j = 1; j < 4; ++j) {
        const floatx4_t p = ((const floatx4_t*)s_t[j])[(ta * T + tw) * 64 + lane];
        v[0] += p[0];
        v[1] += p[1];
        v[2] += p[2];
        v[3] += p[3];
      }
      if (SWAP) {   // lane: row m = r16 of block ta, columns 4 q4 .. +3 of block tw
        const int m = m0 + 16 * ta + r16;
        if (m < M) epilogue4<EPI>(ea, vec, m, n0 + 16 * tw + 4 * q4, N, v);
      } else {
        const int n = n0 + 16 * tw + r16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + 16 * ta + 4 * q4 + r;
          if (m < M && n < N) epilogue<EPI>(ea, m, n, v[r]);
        }
      }
    }
}

// Bytes of one wave's LDS region in k_gemm_sk2 (rounds of 6 or 8 k-steps for
// T = 1 take the larger, 8; T = 2 uses 4).
constexpr int sk2_region_bytes(int T) {
  return T == 1 ? 2 * 16 * (4 * 8 + 1) * 16 : 2 * 32 * (4 * 4 + 1) * 16;
}

bool gemm_skinny_fits(int M, int N, int K, bool rms) {
  return M > 0 && M <= 128 && N > 0 && K % 128 == 0 &&
         (!rms || K / 128 <= (M > 32 ? 12 : SK_KB));
}

hipError_t gemm_skinny(int epi, bool rms, const bf16_t* A, int lda, const bf16_t* W, int M, int N,
                       int K, float eps, const EpiArgs& ea, hipStream_t st) {
  if (!gemm_skinny_fits(M, N, K, rms) || lda % 8) return hipErrorInvalidValue;
  // 32x32 work-group tiles halve the L2 re-reads of A and W; 16x16 tiles give
  // more work-groups.  Measured: 32x32 wins for wide N at 33-64 rows, 16x16
  // for narrow N at 64 rows; above 64 rows 32x32 wins where its grid still
  // has 128 or more work-groups (d 1536 o / proj at 128 rows, 192: 2982
  // against 3186 us per cfg5 step) and loses below (d 768 at 96 / 128 rows,
  // 72 / 96 work-groups: 764.9 -> 708.8, 818.6 -> 764.2 us per step with
  // 16x16).  The RMS projections above 64 rows keep 32x32.
  const long long g2 = (long long)((N + 31) / 32) * ((M + 31) / 32);
  const int T = (M > 64 ? (rms || g2 >= 128) : (M > 32 && N >= 2048)) ? 2 : 1;
  dim3 grid((N + 16 * T - 1) / (16 * T), (M + 16 * T - 1) / (16 * T));
  // batch depth: the wave's whole K quarter when it fits (fewer registers ->
  // more resident work-groups)
  const int kw = K >> 7;
  // LDS-staged variant: rounds of 8 k-steps (16 x 16 tiles) or 4 (32 x 32).
  // With RMS its extra pass over A pays only above 64 rows (measured: cfg5
  // +1.6%, batch 64 -8.5%, batch 16 -4%), and the row sums of squares of a
  // quarter must fit a wave's region.
  if (!rms || (M > 64 && 16 * T * 4 * kw * 4 <= sk2_region_bytes(T))) {
    // 32 x 32 tiles with a whole number of 3-round groups: three rounds in
    // flight per wave (cfg5 decode 3421 -> 3310 us per step, measured); the
    // 16 x 16 tiles measured ~1% slower with it (batch-64 proj: 3 rounds)
    const int xd = T == 2 && kw % 4 == 0 && (kw / 4) % 3 == 0 ? 3 : 1;
#define ANN_SK2_R(E, R)                                                                          \
  if (T == 1) {                                                                                  \
    if (kw <= 6)                                                                                 \
      hipLaunchKernelGGL((k_gemm_sk2<E, R, 6, 1, 1>), grid, dim3(256), 0, st, A, lda, W, M, N,   \
                         K, eps, ea);                                                            \
    else                                                                                         \
      hipLaunchKernelGGL((k_gemm_sk2<E, R, 8, 1, 1>), grid, dim3(256), 0, st, A, lda, W, M, N,   \
                         K, eps, ea);                                                            \
  } else if (xd == 1) {                                                                          \
    hipLaunchKernelGGL((k_gemm_sk2<E, R, 4, 2, 1>), grid, dim3(256), 0, st, A, lda, W, M, N, K,  \
                       eps, ea);                                                                 \
  } else {                                                                                       \
    hipLaunchKernelGGL((k_gemm_sk2<E, R, 4, 2, 3>), grid, dim3(256), 0, st, A, lda, W, M, N, K,  \
                       eps, ea);                                                                 \
  }
#define ANN_SK2(E)       \
  if (rms) {             \
    ANN_SK2_R(E, true)   \
  } else {               \
    ANN_SK2_R(E, false)  \
  }                      \
  break;
    switch (epi) {
      case EPI_STORE: ANN_SK2(EPI_STORE)
      case EPI_RELU2: ANN_SK2(EPI_RELU2)
      case EPI_RESID_ATTN: ANN_SK2(EPI_RESID_ATTN)
      case EPI_RESID_MLP: ANN_SK2(EPI_RESID_MLP)
      case EPI_LOGITS: ANN_SK2(EPI_LOGITS)
      default: return hipErrorInvalidValue;
    }
#undef ANN_SK2
#undef ANN_SK2_R
    return hipGetLastError();
  }
  const int kb = kw <= 6 ? 6 : kw <= 12 ? 12 : SK_KB;
#define ANN_SK_T(E, R, KBV)                                                                   \
  if (T == 1)                                                                                 \
    hipLaunchKernelGGL((k_gemm_sk<E, R, KBV, 1>), grid, dim3(256), 0, st, A, lda, W, M, N, K,  \
                       eps, ea);                                                              \
  else                                                                                        \
    hipLaunchKernelGGL((k_gemm_sk<E, R, (KBV > 12 ? 12 : KBV), 2>), grid, dim3(256), 0, st, A, \
                       lda, W, M, N, K, eps, ea);
#define ANN_SK_KB(E, R)    \
  if (kb == 6) {           \
    ANN_SK_T(E, R, 6)      \
  } else if (kb == 12) {   \
    ANN_SK_T(E, R, 12)     \
  } else {                 \
    ANN_SK_T(E, R, SK_KB)  \
  }
#define ANN_SK(E)            \
  if (rms) {                 \
    ANN_SK_KB(E, true)       \
  } else {                   \
    ANN_SK_KB(E, false)      \
  }                          \
  break;
  switch (epi) {
    case EPI_STORE: ANN_SK(EPI_STORE)
    case EPI_RELU2: ANN_SK(EPI_RELU2)
    case EPI_RESID_ATTN: ANN_SK(EPI_RESID_ATTN)
    case EPI_RESID_MLP: ANN_SK(EPI_RESID_MLP)
    case EPI_LOGITS: ANN_SK(EPI_LOGITS)
    default: return hipErrorInvalidValue;
  }
#undef ANN_SK_KB
#undef ANN_SK_T
#undef ANN_SK
  return hipGetLastError();
}

hipError_t gemm_batched(int epi, const bf16_t* A, int lda, long long sA, const bf16_t* W,
                        long long sW, int M, int N, int K, const EpiArgs& ea, long long sOut,
                        long long sX, int batch, hipStream_t st) {
  if (K % GM_BK != 0 || M <= 0 || N <= 0 || batch <= 0 || batch > 65535)
    return hipErrorInvalidValue;
  const int bm = M <= 64 ? 64 : GM_BM;
  dim3 grid((N + GM_BN - 1) / GM_BN, (M + bm - 1) / bm, batch);
  EpiArgs e2 = ea;
  // symmetric form: square outputs of whole 128 x 128 tiles, 16-byte aligned
  e2.sym = ea.sym && (epi == EPI_STORE || epi == EPI_PE_B) && M == N && bm == GM_BM &&
           M % GM_BM == 0 && ea.ldo % 8 == 0 && ((uintptr_t)ea.out & 15) == 0 &&
           sOut % 8 == 0 && (epi != EPI_PE_B || (ea.ldr % 8 == 0 && sX % 8 == 0 &&
                                                 ((uintptr_t)ea.x & 15) == 0));
  if (e2.sym) {
    const int nb = M / GM_BM;
    grid = dim3(nb * (nb + 1) / 2, 1, batch);
  }
#define ANN_GB(E)                                                                              \
  if (bm == 64)                                                                                \
    hipLaunchKernelGGL((k_gemm_bat<E, 64>), grid, dim3(256), 0, st, A, lda, sA, W, sW, M, N,   \
                       K, e2, sOut, sX);                                                       \
  else                                                                                         \
    hipLaunchKernelGGL((k_gemm_bat<E, GM_BM>), grid, dim3(256), 0, st, A, lda, sA, W, sW, M,   \
                       N, K, e2, sOut, sX);                                                    \
  break;
  switch (epi) {
    case EPI_STORE: ANN_GB(EPI_STORE)
    case EPI_PE_B: ANN_GB(EPI_PE_B)
    case EPI_PE_X: ANN_GB(EPI_PE_X)
    default: return hipErrorInvalidValue;
  }
#undef ANN_GB
  return hipGetLastError();
}

// The fused QKV epilogue needs every 128-column tile inside one section and
// whole heads per tile: d = H * Dh a multiple of 128, Dh 64 or 128.
bool gemm_qkv_fits(int M, int N, int K, const EpiArgs& ea) {
  const int d = ea.H * ea.Dh;
  return M > 0 && K % GM_BK == 0 && (ea.Dh == 64 || ea.Dh == 128) && d % GM_BN == 0 &&
         N == 3 * d && ea.T > 0 && M % ea.T == 0 && ea.ldo % 8 == 0 && ea.out && ea.kc &&
         ea.vc && ea.pos && ea.cs && ea.sn;
}

// Decode projections of 65-128 rows with a plain-store epilogue on 64 x 64
// MFMA tiles (A already normalised).
hipError_t gemm_decode64(int epi, const bf16_t* A, int lda, const bf16_t* W, int M, int N, int K,
                         const EpiArgs& ea, hipStream_t st) {
  if (K % GM_BK != 0 || M <= 0 || N <= 0) return hipErrorInvalidValue;
  dim3 grid((N + 63) / 64, (M + 63) / 64);
  // four K tiles in flight per thread (cfg5 qkv / fc: 3310 -> 3017 us per
  // decode step, measured; eight: 3073)
  const bool deep = (K / GM_BK) % 4 == 0;
#define ANN_D64(E)                                                                               \
  if (!deep)                                                                                     \
    hipLaunchKernelGGL((k_gemm<E, 64, 64>), grid, dim3(256), 0, st, A, lda, W, M, N, K, ea);     \
  else                                                                                           \
    hipLaunchKernelGGL((k_gemm_deep<E, 64, 64, 4>), grid, dim3(256), 0, st, A, lda, W, M, N, K,  \
                       ea);
  if (epi == EPI_STORE) {
    ANN_D64(EPI_STORE)
  } else if (epi == EPI_RELU2) {
    ANN_D64(EPI_RELU2)
  } else {
    return hipErrorInvalidValue;
  }
#undef ANN_D64
  return hipGetLastError();
}

hipError_t gemm(int epi, const bf16_t* A, int lda, const bf16_t* W, int M, int N, int K,
                const EpiArgs& ea, hipStream_t st) {
  if (K % GM_BK != 0 || M <= 0 || N <= 0) return hipErrorInvalidValue;
  // large shapes of the epilogues where it measured faster: the 256 x 256
  // one-work-group-per-CU kernel (gemm_big.hip).  ANN_GEMM_BIG=0 keeps every
  // shape on the tiles below, ANN_GEMM_BIG=2 sends every epilogue it takes
  // there (read at every call)
  const char* big_env = getenv("ANN_GEMM_BIG");
  const int big_mode = big_env ? atoi(big_env) : 1;
  if (big_mode != 0 && (big_mode == 2 || gemm_big_routes(epi, M, N)) &&
      gemm_big_fits(epi, A, lda, M, N, K, ea)) {
    if (epi == EPI_QKV && !gemm_qkv_fits(M, N, K, ea)) return hipErrorInvalidValue;
    return gemm_big(epi, A, lda, W, M, N, K, ea, st);
  }
  // tile: 64 x 128 for at most 64 rows; 128 x 128 below 512 rows; then
  // 256 x 128 (wide outputs, and the 128-column QKV / CE epilogues) or
  // 128 x 256 (outputs of at most 1024 columns: the o / proj projections)
  const int shape = M <= 64 ? 0 : M < 512 ? 1
                  : (epi == EPI_QKV || epi == EPI_CE || N > 1024) ? 2 : 3;
  const int bm = shape == 0 ? 64 : shape == 2 ? 256 : 128;
  const int bn = shape == 3 ? 256 : GM_BN;
  dim3 grid((N + bn - 1) / bn, (M + bm - 1) / bm);
#define ANN_GM_ONE(E, S)                                                                       \
  if (S == 0)                                                                                  \
    hipLaunchKernelGGL((k_gemm<E, 64, GM_BN>), grid, dim3(256), 0, st, A, lda, W, M, N, K, ea); \
  else if (S == 1)                                                                             \
    hipLaunchKernelGGL((k_gemm<E, 128, GM_BN>), grid, dim3(256), 0, st, A, lda, W, M, N, K,    \
                       ea);                                                                    \
  else if (S == 2)                                                                             \
    hipLaunchKernelGGL((k_gemm_2w<E, 256, GM_BN>), grid, dim3(256), 0, st, A, lda, W, M, N, K, \
                       ea);
#define ANN_GM(E)                                                                              \
  ANN_GM_ONE(E, shape)                                                                         \
  else hipLaunchKernelGGL((k_gemm_2w<E, 128, 256>), grid, dim3(256), 0, st, A, lda, W, M, N,   \
                          K, ea);                                                              \
  break;
  switch (epi) {
    case EPI_STORE: ANN_GM(EPI_STORE)
    case EPI_RELU2: ANN_GM(EPI_RELU2)
    case EPI_RESID_ATTN: ANN_GM(EPI_RESID_ATTN)
    case EPI_RESID_MLP: ANN_GM(EPI_RESID_MLP)
    case EPI_LOGITS: ANN_GM(EPI_LOGITS)
    case EPI_QKV:
      if (!gemm_qkv_fits(M, N, K, ea)) return hipErrorInvalidValue;
      ANN_GM_ONE(EPI_QKV, shape)
      break;
    case EPI_CE:
      if (!ea.ce_part || !ea.ce_tz || !ea.tgt || ea.ldz < M) return hipErrorInvalidValue;
      ANN_GM_ONE(EPI_CE, shape)
      break;
    case EPI_TOPK: {
      // decode rows only (the 64- and 128-row tiles); every 128 columns one record
      if (shape > 1 || !ea.cand || !ea.cand_r || ea.nt != (N + 127) / 128 || ea.Vs < 1 ||
          ea.Vs > N || N > 65536 || (ea.logits && ea.ldz < N))
        return hipErrorInvalidValue;
      ANN_GM_ONE(EPI_TOPK, shape)
      break;
    }
    default:
      return hipErrorInvalidValue;
  }
#undef ANN_GM
#undef ANN_GM_ONE
  return hipGetLastError();
}

}  // namespace ann
