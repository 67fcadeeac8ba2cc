// Sampling of one token per row from bf16 z = lm_head logits before the
// softcap (sample.py:44-49):
//   greedy (temperature 0): argmax of z over the first Vs entries, lowest
//     index on ties (softcap is increasing, so this is the argmax of the
//     softcapped logits);
//   otherwise: zc = softcap(z) / temperature; kth = k-th largest zc; keep
//     every zc >= kth (ties included, as `where(z < kth, -1e9, z)`); draw
//     u ~ U[0,1) from Philox4x32-10 and return the first kept index whose
//     running sum of exp(zc - max) exceeds u * total.
// The k-th largest is found by a binary search over the 16-bit ordered keys
// of z (count of keys >= T per round); one work-group per row.
#include <math.h>
#include "common.h"
#include "launch.h"

namespace ann {

constexpr int SMP_THREADS = 1024;

__device__ __forceinline__ uint32_t okey(bf16_t h) {  // order-preserving 16-bit key
  return (h & 0x8000u) ? (uint32_t)(~h & 0xffffu) : (uint32_t)(h | 0x8000u);
}

__device__ __forceinline__ uint32_t mulhilo(uint32_t a, uint32_t b, uint32_t* hi) {
  const uint64_t p = (uint64_t)a * b;
  *hi = (uint32_t)(p >> 32);
  return (uint32_t)p;
}

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11): first output word.
__device__ uint32_t philox_x(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0,
                             uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    uint32_t hi0, hi1;
    const uint32_t lo0 = mulhilo(0xD2511F53u, c0, &hi0);
    const uint32_t lo1 = mulhilo(0xCD9E8D57u, c2, &hi1);
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c0;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)v, o, 64);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), o, 64);
    const uint64_t w = ((uint64_t)hi << 32) | lo;
    v = w > v ? w : v;
  }
  return v;
}

constexpr int SMP_CH = 7;  // 16-byte chunks per thread: 1024 * 56 >= 50257

__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t* red) {
  v = wave_max_u64(v);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wv] = v;
  __syncthreads();
  uint64_t b = 0;
#pragma unroll
  for (int w = 0; w < SMP_THREADS / 64; ++w) b = red[w] > b ? red[w] : b;
  return b;
}

// One work-group per row; thread t holds the contiguous slice
// [56 t, 56 t + 56) of the row in registers, so the row is read from memory
// once and every pass (radix select, max, weights, scan, draw) runs on
// registers and LDS.
__global__ __launch_bounds__(SMP_THREADS) void k_sample(const bf16_t* __restrict__ zall, int ldz,
                                                        int Vs, const SampParams* __restrict__ sp,
                                                        unsigned long long* __restrict__ steps,
                                                        int32_t* __restrict__ out_tok,
                                                        int32_t* __restrict__ pos, int pos_adv) {
  const float temperature = sp->temperature;
  const int top_k = sp->top_k;
  const uint64_t seed = sp->seed;
  __shared__ uint32_t s_cnt[2][SMP_THREADS / 64];
  __shared__ uint64_t s_red[SMP_THREADS / 64];
  __shared__ float s_wsum[SMP_THREADS / 64];
  __shared__ uint32_t s_misc[4];
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const bf16_t* z = zall + (size_t)row * ldz;
  const int base = tid * SMP_CH * 8;

  uint4 raw[SMP_CH];
#pragma unroll
  for (int c = 0; c < SMP_CH; ++c)
    raw[c] = (base + c * 8 < ldz) ? *(const uint4*)(z + base + c * 8) : make_uint4(0, 0, 0, 0);
  auto elem = [&](int i) -> bf16_t {   // i in [0, 56)
    const uint4& w = raw[i >> 3];
    const uint32_t word = (i & 7) < 2 ? w.x : (i & 7) < 4 ? w.y : (i & 7) < 6 ? w.z : w.w;
    return (bf16_t)((i & 1) ? (word >> 16) : (word & 0xffffu));
  };

  if (temperature == 0.f) {
    uint64_t best = 0;
#pragma unroll
    for (int i = 0; i < SMP_CH * 8; ++i) {
      const int gi = base + i;
      if (gi < Vs) {
        const uint64_t key = ((uint64_t)okey(elem(i)) << 32) | (uint64_t)(0xffffffffu - (uint32_t)gi);
        best = key > best ? key : best;
      }
    }
    best = block_max_u64(best, s_red);
    if (tid == 0) {
      out_tok[row] = (int32_t)(0xffffffffu - (uint32_t)(best & 0xffffffffu));
      if (pos) pos[row] += pos_adv;
    }
    return;
  }

  // ---- maximum key, then the k-th largest key (exact) when top-k applies:
  // binary search for the largest T with count(key >= T) >= top_k; each
  // round counts from registers and reduces once over the work-group
  uint32_t kmax = 0;
#pragma unroll
  for (int i = 0; i < SMP_CH * 8; ++i)
    if (base + i < Vs) kmax = max(kmax, okey(elem(i)));
  kmax = (uint32_t)block_max_u64(kmax, s_red);
  uint32_t thr_key = 0;
  const bool use_thr = top_k > 0 && top_k < Vs;
  if (use_thr) {
    uint32_t lo = 0, hi = kmax;
    int round = 0;
    while (lo < hi) {
      const uint32_t mid = (lo + hi + 1) >> 1;
      uint32_t c = 0;
#pragma unroll
      for (int i = 0; i < SMP_CH * 8; ++i) c += (base + i < Vs && okey(elem(i)) >= mid) ? 1u : 0u;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o, 64);
      uint32_t* cb = s_cnt[round & 1];
      if (lane == 0) cb[wv] = c;
      __syncthreads();
      uint32_t tot = 0;
#pragma unroll
      for (int w = 0; w < SMP_THREADS / 64; ++w) tot += cb[w];
      if (tot >= (uint32_t)top_k) lo = mid;
      else hi = mid - 1;
      ++round;
    }
    thr_key = lo;
  }
  // ---- threshold and maximum in the softcapped / tempered domain
  auto key2bf = [](uint32_t k) -> bf16_t {
    return (bf16_t)((k & 0x8000u) ? (k & 0x7fffu) : (~k & 0xffffu));
  };
  const float tmp = temperature;
  const float zmax = softcap(bf2f(key2bf(kmax))) / tmp;
  const float zthr = use_thr ? softcap(bf2f(key2bf(thr_key))) / tmp : -INFINITY;
  // softcap / temperature is non-decreasing in z, so "kept" (zc >= zthr) is
  // "key >= thr_key" unless the value just below the threshold rounds to the
  // same zc (saturated softcap): checked once, exact fallback otherwise.
  const bool by_key = !use_thr || thr_key == 0 ||
                      softcap(bf2f(key2bf(thr_key - 1))) / tmp < zthr;
  auto kept = [&](int i) -> bool {
    if (base + i >= Vs) return false;
    const bf16_t h = elem(i);
    return by_key ? okey(h) >= thr_key : softcap(bf2f(h)) / tmp >= zthr;
  };

  // ---- weights of this thread's slice, block exclusive scan (fixed order)
  float local = 0.f;
#pragma unroll
  for (int i = 0; i < SMP_CH * 8; ++i)
    if (kept(i)) local += expf(softcap(bf2f(elem(i))) / tmp - zmax);
  float incl = local;   // inclusive scan within the wave
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float v = __shfl_up(incl, o, 64);
    if (lane >= o) incl += v;
  }
  if (lane == 63) s_wsum[wv] = incl;
  __syncthreads();
  float wbase = 0.f, total = 0.f;
  for (int w = 0; w < SMP_THREADS / 64; ++w) {
    if (w < wv) wbase += s_wsum[w];
    total += s_wsum[w];
  }
  const float before = wbase + incl - local;
  const uint64_t step = steps[row];
  const uint32_t rw = philox_x((uint32_t)step, (uint32_t)row, (uint32_t)(step >> 32), 0u,
                               (uint32_t)seed, (uint32_t)(seed >> 32));
  const float target = (float)(rw >> 8) * (1.0f / 16777216.0f) * total;
  if (tid == 0) s_misc[0] = 0xffffffffu;
  __syncthreads();
  if (local > 0.f && target >= before && target < before + local) {
    float run = before;
    int pick = -1, last = -1;
#pragma unroll
    for (int i = 0; i < SMP_CH * 8; ++i) {
      if (pick < 0 && kept(i)) {
        last = base + i;
        run += expf(softcap(bf2f(elem(i))) / tmp - zmax);
        if (target < run) pick = base + i;
      }
    }
    if (pick < 0) pick = last;
    atomicMin(&s_misc[0], (uint32_t)pick);
  }
  __syncthreads();
  if (s_misc[0] == 0xffffffffu) {
    // rounding put the target at/after the total: take the last kept index
    int lastk = -1;
#pragma unroll
    for (int i = 0; i < SMP_CH * 8; ++i)
      if (kept(i)) lastk = base + i;
    __syncthreads();
    if (tid == 0) s_misc[2] = 0;
    __syncthreads();
    if (lastk >= 0) atomicMax(&s_misc[2], (uint32_t)lastk);
    __syncthreads();
    if (tid == 0) s_misc[0] = s_misc[2];
  }
  if (tid == 0) {
    out_tok[row] = (int32_t)s_misc[0];
    if (pos) pos[row] += pos_adv;
    steps[row] = step + 1;
  }
}

__global__ void k_set_sampling(SampParams* sp, unsigned long long* steps, int B, float temperature,
                               int top_k, unsigned long long seed, unsigned long long step) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i == 0) {
    sp->temperature = temperature;
    sp->top_k = top_k;
    sp->seed = seed;
  }
  if (i < B) steps[i] = step;
}

__global__ void k_set_pos(int32_t* pos, int B, int value) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < B) pos[i] = value;
}

__global__ void k_advance_pos(int32_t* pos, int B, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < B) pos[i] += n;
}

hipError_t sample(const bf16_t* z, int ldz, int B, int Vs, const SampParams* sp,
                  unsigned long long* steps, int32_t* out_tok, int32_t* pos, int pos_adv,
                  hipStream_t st) {
  hipLaunchKernelGGL(k_sample, dim3(B), dim3(SMP_THREADS), 0, st, z, ldz, Vs, sp, steps, out_tok,
                     pos, pos_adv);
  return hipGetLastError();
}

hipError_t set_sampling(SampParams* sp, unsigned long long* steps, int B, float temperature,
                        int top_k, unsigned long long seed, unsigned long long step,
                        hipStream_t st) {
  hipLaunchKernelGGL(k_set_sampling, dim3((B + 255) / 256), dim3(256), 0, st, sp, steps, B,
                     temperature, top_k, seed, step);
  return hipGetLastError();
}

hipError_t set_pos(int32_t* pos, int B, int value, hipStream_t st) {
  hipLaunchKernelGGL(k_set_pos, dim3((B + 255) / 256), dim3(256), 0, st, pos, B, value);
  return hipGetLastError();
}

hipError_t advance_pos(int32_t* pos, int B, int n, hipStream_t st) {
  hipLaunchKernelGGL(k_advance_pos, dim3((B + 255) / 256), dim3(256), 0, st, pos, B, n);
  return hipGetLastError();
}

}  // namespace ann
