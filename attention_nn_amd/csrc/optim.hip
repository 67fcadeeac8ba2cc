// Optimizer step of the training loop: MuonAdam (muon.py:66-137) and its
// fused kernels (metal_kernels.py:236-328).
//
//  * k_adam, k_muon_momentum, k_muon_apply: fp32 elementwise, 16-byte
//    accesses, HBM-bound.  Same arithmetic and the same comparisons (cautious
//    weight decay) as the reference kernels.
//  * Polar Express (muon.py:28-44) on a batch of (M, N) matrices: x = bf16(g /
//    (||g||_F * 1.02 + 1e-6)), then five iterations of bf16 products on the
//    MFMA GEMM (batched over blockIdx.z).  Every product is an "NT" GEMM of
//    k_gemm: x x^T directly; A A because A is symmetric; B x through one
//    transpose of x per iteration (x B for tall matrices, B symmetric).  The
//    combinations b A + c A^2 and a x + B x run in the GEMM epilogues with the
//    eager rounding of each op.
//  * NorMuon (muon.py:47-63): mean of squares along the reduced axis, one
//    work-group per matrix for the norms and the second-moment update, then
//    the broadcast scale.
// All reductions run in a fixed order: results are bit-reproducible.
#include <math.h>
#include <string.h>
#include <mutex>
#include "common.h"
#include "launch.h"

namespace ann {

namespace {
unsigned grid_for(size_t n, unsigned threads) {
  size_t g = (n + threads - 1) / threads;
  if (g > 65536) g = 65536;
  return g ? (unsigned)g : 1u;
}
}  // namespace

// ---- elementwise --------------------------------------------------------------

// adam_step (metal_kernels.py:241-259): fp32 moments, cautious weight decay.
__device__ __forceinline__ void adam1(float pv, float gv, float m, float v, float b1, float b2,
                                      float eps, float step, float wd, float& po, float& mo,
                                      float& vo) {
  const float mv = b1 * m + (1.0f - b1) * gv;
  const float vv = b2 * v + (1.0f - b2) * gv * gv;
  float u = mv / (sqrtf(vv) + eps) * step;
  if (u * pv > 0.0f) u += pv * wd;
  po = pv - u;
  mo = mv;
  vo = vv;
}

__global__ void k_adam(const float* __restrict__ p, const float* __restrict__ g,
                       const float* __restrict__ m, const float* __restrict__ v, size_t n,
                       float b1, float b2, float eps, float step, float wd, float* __restrict__ po,
                       float* __restrict__ mo, float* __restrict__ vo) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    adam1(p[i], g[i], m[i], v[i], b1, b2, eps, step, wd, po[i], mo[i], vo[i]);
}

// muon_momentum (metal_kernels.py:277-290): buf <- lerp(buf, g, 1 - mu),
// geff <- lerp(g, buf, mu).
__global__ void k_muon_momentum(const float* __restrict__ g, const float* __restrict__ buf,
                                size_t n, float mu, float* __restrict__ geff,
                                float* __restrict__ bo) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float gv = g[i], b = buf[i];
    const float bv = b + (1.0f - mu) * (gv - b);
    bo[i] = bv;
    geff[i] = gv + mu * (bv - gv);
  }
}

// muon_apply (metal_kernels.py:306-319): decay where u and p agree in sign.
__global__ void k_muon_apply(const float* __restrict__ p, const float* __restrict__ u, size_t n,
                             float lr, float wd, float* __restrict__ po) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float uv = u[i];
    float pv = p[i];
    if (uv * pv >= 0.0f) pv -= pv * wd * lr;
    po[i] = pv - uv * lr;
  }
}

// ---- Polar Express ------------------------------------------------------------

constexpr int PE_CHUNK = 8192;   // elements per partial sum of squares
constexpr int PE_THREADS = 256;   // a thread reads 8 float4 of a chunk

// Partial sums of squares: block (chunk c, matrix z), eight independent
// 16-byte loads per thread, then a fixed-order tree.  mn % 4 == 0 (M, N are
// multiples of 64).
__global__ __launch_bounds__(PE_THREADS) void k_pe_sumsq(const float* __restrict__ g, size_t mn,
                                                         int nch, float* __restrict__ part) {
  __shared__ float red[PE_THREADS];
  const int c = blockIdx.x, z = blockIdx.y, tid = threadIdx.x;
  const float4* gz = (const float4*)(g + (size_t)z * mn);
  const size_t q0 = (size_t)c * (PE_CHUNK / 4), q1 = min(mn / 4, q0 + PE_CHUNK / 4);
  float4 v[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const size_t i = q0 + tid + (size_t)u * PE_THREADS;
    v[u] = i < q1 ? gz[i] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < 8; ++u) s += ((v[u].x * v[u].x + v[u].y * v[u].y) + v[u].z * v[u].z) + v[u].w * v[u].w;
  red[tid] = s;
  __syncthreads();
  for (int w = PE_THREADS / 2; w > 0; w >>= 1) {
    if (tid < w) red[tid] += red[tid + w];
    __syncthreads();
  }
  if (tid == 0) part[(size_t)z * nch + c] = red[0];
}

// den[z] = sqrt(sum of the partials) * 1.02 + 1e-6, one wave per matrix,
// lane-strided then a fixed-order wave reduction.
__global__ __launch_bounds__(64) void k_pe_norm(const float* __restrict__ part, int nch,
                                                float* __restrict__ den) {
  const int z = blockIdx.x, lane = threadIdx.x;
  float s = 0.f;
  for (int c = lane; c < nch; c += 64) s += part[(size_t)z * nch + c];
  s = wave_sum(s);
  if (lane == 0) den[z] = sqrtf(s) * 1.02f + 1e-6f;
}

// x = bf16(g / den), four elements per thread.
__global__ void k_pe_scale(const float* __restrict__ g, size_t mn, const float* __restrict__ den,
                           bf16_t* __restrict__ x) {
  const int z = blockIdx.y;
  const float dz = den[z];
  const float4* gz = (const float4*)(g + (size_t)z * mn);
  uint2* xz = (uint2*)(x + (size_t)z * mn);
  const size_t n4 = mn / 4, stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
    const float4 v = gz[i];
    xz[i] = make_uint2(pack2(v.x / dz, v.y / dz), pack2(v.z / dz, v.w / dz));
  }
}

// dst (C, R) = src (R, C)^T per matrix, 64 x 64 tiles through LDS.
constexpr int TR_T = 64;
__global__ __launch_bounds__(256) void k_transpose_bf16(const bf16_t* __restrict__ src,
                                                        bf16_t* __restrict__ dst, int R, int C) {
  __shared__ bf16_t t[TR_T][TR_T + 2];
  const int z = blockIdx.z;
  const int r0 = blockIdx.y * TR_T, c0 = blockIdx.x * TR_T;
  const bf16_t* s = src + (size_t)z * R * C;
  bf16_t* d = dst + (size_t)z * R * C;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int i = ty; i < TR_T; i += 4) {
    const int r = r0 + i, c = c0 + tx;
    t[i][tx] = (r < R && c < C) ? s[(size_t)r * C + c] : (bf16_t)0;
  }
  __syncthreads();
  for (int i = ty; i < TR_T; i += 4) {
    const int c = c0 + i, r = r0 + tx;
    if (c < C && r < R) d[(size_t)c * R + r] = t[tx][i];
  }
}

// Polar Express coefficients (muon.py:19-25; num_iters 5, safety 2e-2, cushion 2).
constexpr double PE_COEF[5][3] = {
    {8.156554524902461, -22.48329292557795, 15.878769915207462},
    {4.042929935166739, -2.808917465908714, 0.5000178451051316},
    {3.8916678022926607, -2.772484153217685, 0.5060648178503393},
    {3.285753657755655, -2.3681294933425376, 0.46449024233003106},
    {2.3465413258596377, -1.7097828382687081, 0.42323551169305323},
};

namespace {
// The eager bf16 ops of the reference multiply by a Python float, which a
// bf16 array takes in its own dtype: the coefficient enters as bf16.
float bf16_round_host(double v) {
  float f = (float)v;
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  memcpy(&f, &u, 4);
  return f;
}
size_t up256(size_t v) { return (v + 255) / 256 * 256; }
}  // namespace

size_t polar_express_ws_bytes(int batch, int M, int N) {
  if (batch <= 0 || M <= 0 || N <= 0) return 0;
  const size_t mn = (size_t)M * N, S = M < N ? M : N;
  const size_t nch = (mn + PE_CHUNK - 1) / PE_CHUNK;
  return up256(batch * mn * 2) * 3 + up256(batch * S * S * 2) * 2 + up256(batch * nch * 4) +
         up256(batch * 4);
}

hipError_t polar_express(const float* g, int batch, int M, int N, bf16_t* out, void* ws,
                         size_t ws_bytes, hipStream_t st) {
  if (batch <= 0 || batch > 65535 || M <= 0 || N <= 0 || M % 64 || N % 64 || !g || !out ||
      !ws || ws_bytes < polar_express_ws_bytes(batch, M, N))
    return hipErrorInvalidValue;
  const size_t mn = (size_t)M * N, S = M < N ? M : N;
  const int nch = (int)((mn + PE_CHUNK - 1) / PE_CHUNK);
  char* w = (char*)ws;
  bf16_t* xb = (bf16_t*)w;  w += up256(batch * mn * 2);    // the other x buffer
  bf16_t* xt = (bf16_t*)w;  w += up256(batch * mn * 2);    // x^T of the current x
  bf16_t* xt2 = (bf16_t*)w; w += up256(batch * mn * 2);    // x^T of the next x
  bf16_t* am = (bf16_t*)w;  w += up256(batch * S * S * 2); // A
  bf16_t* bm = (bf16_t*)w;  w += up256(batch * S * S * 2); // B
  float* part = (float*)w;  w += up256(batch * (size_t)nch * 4);
  float* den = (float*)w;
  // x0 goes to xb so that the fifth (odd) iteration lands in out
  hipLaunchKernelGGL(k_pe_sumsq, dim3(nch, batch), dim3(PE_THREADS), 0, st, g, mn, nch, part);
  hipLaunchKernelGGL(k_pe_norm, dim3(batch), dim3(64), 0, st, part, nch, den);
  const unsigned sg = grid_for(mn / 4, 256);
  hipLaunchKernelGGL(k_pe_scale, dim3(sg < 1024 ? sg : 1024, batch), dim3(256), 0, st, g, mn, den,
                     xb);
  bf16_t* cur = xb;
  bf16_t* nxt = out;
  const bool tall = M > N;
  const dim3 tg((N + TR_T - 1) / TR_T, (M + TR_T - 1) / TR_T, batch);
  // x^T of the first x by a transpose; each iteration's x' = a x + B x
  // epilogue also writes x'^T for the next one (the last one's is not needed)
  hipLaunchKernelGGL(k_transpose_bf16, tg, dim3(256), 0, st, cur, xt, M, N);
  for (int it = 0; it < 5; ++it) {
    const float a = bf16_round_host(PE_COEF[it][0]);
    const float b = bf16_round_host(PE_COEF[it][1]);
    const float c = bf16_round_host(PE_COEF[it][2]);
    EpiArgs ea{};
    hipError_t e;
    if (!tall) {
      // A = x x^T (M x M, K = N); A and B below are symmetric: only the tiles
      // on and above the diagonal are computed (their mirrors stored transposed)
      ea.out = am;
      ea.ldo = M;
      ea.sym = 1;
      e = gemm_batched(EPI_STORE, cur, N, (long long)mn, cur, (long long)mn, M, M, N, ea,
                       (long long)S * S, 0, batch, st);
      if (e != hipSuccess) return e;
      // B = b A + c (A A)
      ea.out = bm;
      ea.x = am;
      ea.ldr = M;
      ea.s0 = b;
      ea.s1 = c;
      e = gemm_batched(EPI_PE_B, am, M, (long long)S * S, am, (long long)S * S, M, M, M, ea,
                       (long long)S * S, (long long)S * S, batch, st);
      if (e != hipSuccess) return e;
      // x' = a x + B x: B (M x M) against x^T (N x M)
      ea.sym = 0;
      ea.out = nxt;
      ea.ldo = N;
      ea.x = cur;
      ea.ldr = N;
      ea.s0 = a;
      ea.outT = it < 4 ? xt2 : nullptr;
      ea.ldoT = M;
      e = gemm_batched(EPI_PE_X, bm, M, (long long)S * S, xt, (long long)mn, M, N, M, ea,
                       (long long)mn, (long long)mn, batch, st);
      if (e != hipSuccess) return e;
    } else {
      // A = x^T x (N x N, K = M) from x^T (N x M); A and B symmetric as above
      ea.out = am;
      ea.ldo = N;
      ea.sym = 1;
      e = gemm_batched(EPI_STORE, xt, M, (long long)mn, xt, (long long)mn, N, N, M, ea,
                       (long long)S * S, 0, batch, st);
      if (e != hipSuccess) return e;
      ea.out = bm;
      ea.x = am;
      ea.ldr = N;
      ea.s0 = b;
      ea.s1 = c;
      e = gemm_batched(EPI_PE_B, am, N, (long long)S * S, am, (long long)S * S, N, N, N, ea,
                       (long long)S * S, (long long)S * S, batch, st);
      if (e != hipSuccess) return e;
      ea.sym = 0;
      // x' = a x + x B (B symmetric: its rows are the columns of B)
      ea.out = nxt;
      ea.ldo = N;
      ea.x = cur;
      ea.ldr = N;
      ea.s0 = a;
      ea.outT = it < 4 ? xt2 : nullptr;
      ea.ldoT = M;
      e = gemm_batched(EPI_PE_X, cur, N, (long long)mn, bm, (long long)S * S, M, N, N, ea,
                       (long long)mn, (long long)mn, batch, st);
      if (e != hipSuccess) return e;
    }
    bf16_t* t = cur;
    cur = nxt;
    nxt = t;
    t = xt;
    xt = xt2;
    xt2 = t;
  }
  return hipGetLastError();
}

// ---- NorMuon ------------------------------------------------------------------

// Mean of v^2 along the reduced axis: per row when M >= N (one wave per
// row), per column otherwise (one thread per column, rows in order).
__global__ __launch_bounds__(256) void k_nm_mean_rows(const bf16_t* __restrict__ v, int M, int N,
                                                      float* __restrict__ vm) {
  const int z = blockIdx.y;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= M) return;
  const bf16_t* r = v + ((size_t)z * M + row) * N;
  float s = 0.f;
  for (int j = lane; j < N; j += 64) {
    const float f = bf2f(r[j]);
    s += f * f;
  }
  s = wave_sum(s);
  if (lane == 0) vm[(size_t)z * M + row] = s / (float)N;
}

// Columns: a work-group per 64-column strip, lane = column; its four waves
// take rows w, w + 4, ... (one 128-byte row segment per wave load) and their
// sums are added in wave order.
__global__ __launch_bounds__(256) void k_nm_mean_cols(const bf16_t* __restrict__ v, int M, int N,
                                                      float* __restrict__ vm) {
  __shared__ float q[4][64];
  const int z = blockIdx.y, lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int col = blockIdx.x * 64 + lane;
  const bf16_t* c = v + (size_t)z * M * N + col;
  float s = 0.f;
  if (col < N) {
    int i = wv;
    for (; i + 12 < M; i += 16) {   // four rows in flight per lane
      const float f0 = bf2f(c[(size_t)i * N]), f1 = bf2f(c[(size_t)(i + 4) * N]);
      const float f2 = bf2f(c[(size_t)(i + 8) * N]), f3 = bf2f(c[(size_t)(i + 12) * N]);
      s += f0 * f0;
      s += f1 * f1;
      s += f2 * f2;
      s += f3 * f3;
    }
    for (; i < M; i += 4) {
      const float f = bf2f(c[(size_t)i * N]);
      s += f * f;
    }
  }
  q[wv][lane] = s;
  __syncthreads();
  if (wv == 0 && col < N)
    vm[(size_t)z * N + col] = (((q[0][lane] + q[1][lane]) + q[2][lane]) + q[3][lane]) / (float)M;
}

// One work-group per matrix: v_norm, the second-moment update, the step
// sizes and the final per-line scale (muon.py:55-62).
constexpr int NM_THREADS = 1024;
__global__ __launch_bounds__(NM_THREADS) void k_nm_scale(const float* __restrict__ vm, int R,
                                                        int red, float beta2,
                                                        float* __restrict__ sm,
                                                        float* __restrict__ scale) {
  __shared__ float buf[NM_THREADS];
  const int z = blockIdx.x, tid = threadIdx.x;
  const float* vz = vm + (size_t)z * R;
  float* sz = sm + (size_t)z * R;
  float* cz = scale + (size_t)z * R;
  auto block_sum = [&](float x) {
    buf[tid] = x;
    __syncthreads();
    for (int w = NM_THREADS / 2; w > 0; w >>= 1) {
      if (tid < w) buf[tid] += buf[tid + w];
      __syncthreads();
    }
    const float r = buf[0];
    __syncthreads();
    return r;
  };
  float s = 0.f;
  for (int i = tid; i < R; i += NM_THREADS) s += vz[i];
  const float v_norm = sqrtf(block_sum(s) * (float)red);
  float q = 0.f;
  for (int i = tid; i < R; i += NM_THREADS) {
    const float m2 = sz[i] + (1.0f - beta2) * (vz[i] - sz[i]);
    sz[i] = m2;
    const float stp = rsqrtf(fmaxf(m2, 1e-10f));
    cz[i] = stp;
    q += (vz[i] * (float)red) * (stp * stp);
  }
  const float v_norm_new = sqrtf(block_sum(q));
  const float ratio = v_norm / fmaxf(v_norm_new, 1e-10f);
  for (int i = tid; i < R; i += NM_THREADS) cz[i] = cz[i] * ratio;
}

__global__ void k_nm_apply(const bf16_t* __restrict__ v, int M, int N, int rows,
                           const float* __restrict__ scale, float* __restrict__ out, int batch) {
  const size_t mn = (size_t)M * N, n = mn * batch;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const size_t z = i / mn, e = i - z * mn;
    const size_t line = rows ? e / N : e % N;
    out[i] = bf2f(v[i]) * scale[z * (rows ? M : N) + line];
  }
}

size_t normuon_ws_bytes(int batch, int M, int N) {
  const size_t R = M >= N ? M : N;
  return batch > 0 ? 2 * up256((size_t)batch * R * 4) : 0;
}

hipError_t normuon(const bf16_t* v, float* second_mom, int batch, int M, int N, float beta2,
                   float* out, void* ws, size_t ws_bytes, hipStream_t st) {
  if (batch <= 0 || M <= 0 || N <= 0 || !v || !second_mom || !out || !ws ||
      ws_bytes < normuon_ws_bytes(batch, M, N))
    return hipErrorInvalidValue;
  const bool rows = M >= N;
  const int R = rows ? M : N, red = rows ? N : M;
  float* vm = (float*)ws;
  float* sc = (float*)((char*)ws + up256((size_t)batch * R * 4));
  if (rows)
    hipLaunchKernelGGL(k_nm_mean_rows, dim3((M + 3) / 4, batch), dim3(256), 0, st, v, M, N, vm);
  else
    hipLaunchKernelGGL(k_nm_mean_cols, dim3((N + 63) / 64, batch), dim3(256), 0, st, v, M, N,
                       vm);
  hipLaunchKernelGGL(k_nm_scale, dim3(batch), dim3(NM_THREADS), 0, st, vm, R, red, beta2,
                     second_mom, sc);
  hipLaunchKernelGGL(k_nm_apply, dim3(grid_for((size_t)batch * M * N, 256)), dim3(256), 0, st, v,
                     M, N, (int)rows, sc, out, batch);
  return hipGetLastError();
}

hipError_t adam_step(const float* p, const float* g, const float* m, const float* v, size_t n,
                     float b1, float b2, float eps, float step, float wd, float* po, float* mo,
                     float* vo, hipStream_t st) {
  if (!n) return hipSuccess;
  hipLaunchKernelGGL(k_adam, dim3(grid_for(n, 256)), dim3(256), 0, st, p, g, m, v, n, b1, b2, eps,
                     step, wd, po, mo, vo);
  return hipGetLastError();
}

hipError_t muon_momentum(const float* g, const float* buf, size_t n, float mu, float* geff,
                         float* bo, hipStream_t st) {
  if (!n) return hipSuccess;
  hipLaunchKernelGGL(k_muon_momentum, dim3(grid_for(n, 256)), dim3(256), 0, st, g, buf, n, mu,
                     geff, bo);
  return hipGetLastError();
}

hipError_t muon_apply(const float* p, const float* u, size_t n, float lr, float wd, float* po,
                      hipStream_t st) {
  if (!n) return hipSuccess;
  hipLaunchKernelGGL(k_muon_apply, dim3(grid_for(n, 256)), dim3(256), 0, st, p, u, n, lr, wd, po);
  return hipGetLastError();
}

}  // namespace ann

// ---- NorMuon without an allocation ------------------------------------------
// The scratch of normuon_noalloc (the (batch, R) means and scales) lives in a
// file-scope device array of fixed size: every GPU the library runs on holds
// its own copy until the process ends.  In host code `scratch` names a
// host-side stand-in, not a device address: its address on the current device
// comes from hipGetSymbolAddress, taken once per device with that device
// current, and only that pointer is handed to the kernels.  Every call on one
// GPU shares its array (NorMuon writes all of it before reading it, so nothing
// needs clearing); calls that overlap on one GPU race.
static __device__ __align__(256) unsigned char scratch[ann::NM_SCRATCH_BYTES];

namespace ann {
namespace {
constexpr int NM_MAX_DEVICES = 64;
std::mutex g_nm_mu;
void* g_nm_scratch[NM_MAX_DEVICES];   // device address of `scratch`, per device
}  // namespace

// Device address of this GPU's scratch array; the stream must belong to the
// current device.
hipError_t normuon_scratch(hipStream_t st, void** out) {
  int dev = -1, sdev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  e = hipStreamGetDevice(st, &sdev);
  if (e != hipSuccess) return e;
  if (dev != sdev || dev < 0 || dev >= NM_MAX_DEVICES) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_nm_mu);
  if (!g_nm_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_nm_scratch[dev] = p;
  }
  *out = g_nm_scratch[dev];
  return hipSuccess;
}

hipError_t normuon_noalloc(const bf16_t* v, float* second_mom, int batch, int M, int N,
                           float beta2, float* out, hipStream_t st) {
  if (normuon_ws_bytes(batch, M, N) > NM_SCRATCH_BYTES) return hipErrorInvalidValue;
  void* ws = nullptr;
  const hipError_t e = normuon_scratch(st, &ws);
  if (e != hipSuccess) return e;
  return normuon(v, second_mom, batch, M, N, beta2, out, ws, NM_SCRATCH_BYTES, st);
}

}  // namespace ann
