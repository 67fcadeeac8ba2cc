// Shared device helpers for the gfx950 kernels: bf16 storage as raw 16-bit
// words, round-to-nearest-even conversion, wave64 reductions.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define ANN_WAVE 64

typedef uint16_t bf16_t;

__device__ __forceinline__ float bf2f(bf16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}

// fp32 -> bf16, round to nearest even (gfx950 v_cvt_pk_bf16_f32; equal to
// the bit-level RNE u + 0x7fff + lsb for every non-NaN input, denormals
// included); NaN stays a quiet NaN.
typedef __bf16 bf16x2_hw __attribute__((ext_vector_type(2)));
typedef float floatx2_hw __attribute__((ext_vector_type(2)));
__device__ __forceinline__ bf16_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// Round an fp32 value to the nearest bf16 and widen it back.
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

__device__ __forceinline__ void unpack8(const uint4& w, float* o) {
  o[0] = __uint_as_float(w.x << 16); o[1] = __uint_as_float(w.x & 0xffff0000u);
  o[2] = __uint_as_float(w.y << 16); o[3] = __uint_as_float(w.y & 0xffff0000u);
  o[4] = __uint_as_float(w.z << 16); o[5] = __uint_as_float(w.z & 0xffff0000u);
  o[6] = __uint_as_float(w.w << 16); o[7] = __uint_as_float(w.w & 0xffff0000u);
}

__device__ __forceinline__ uint32_t pack2(float a, float b) {
  const floatx2_hw v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_hw));
}

template <int W>
__device__ __forceinline__ float group_sum(float v) {
  // butterfly over groups of W consecutive lanes (W a power of two <= 64)
#pragma unroll
  for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, W);
  return v;
}

// Sum over a whole wave in a fixed order with DPP row operations (device
// library wavefront reduction); every lane gets the total.
extern "C" __device__ float __ockl_wfred_add_f32(float);
__device__ __forceinline__ float wave_sum(float v) { return __ockl_wfred_add_f32(v); }

// Sum over each group of 4 consecutive lanes (DPP quad permutes).
__device__ __forceinline__ float quad_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1,
                                                            0xf, 0xf, false));   // [1,0,3,2]
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E,
                                                            0xf, 0xf, false));   // [2,3,0,1]
  return v;
}

template <int W>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = W / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, W));
  return v;
}

// Sum over a whole work-group; `red` is LDS scratch of >= blockDim/64 floats.
// Every thread gets the total.  Fixed reduction order: deterministic.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = group_sum<64>(v);
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; ++i) t += red[i];
  return t;
}

// Softcap with the hardware exp2 and reciprocal (a few fp32 ulps from the IEEE
// form): the sampler's weights (its threshold comparisons use the IEEE form)
// and the training loss's sums; the fp32 logits handed out use softcap().
__device__ __forceinline__ float softcap_fast(float z) {
  const float e = __builtin_amdgcn_exp2f((z + 5.0f) * -0.19235933878519512f);  // -log2(e) / 7.5
  return 23.0f * __builtin_amdgcn_rcpf(1.0f + e);
}
// Softcap of the logits: 23 * sigmoid((z + 5) / 7.5).
__device__ __forceinline__ float softcap(float z) {
  float t = (z + 5.0f) / 7.5f;
  return 23.0f * (1.0f / (1.0f + expf(-t)));
}

// Block epilogues of model.py, each eager op rounded to bf16 (y: fp32
// accumulator of the projection, lam: the layer's r0 r1 p0 p1 x0l).
//   x = ((r0 x) + (p0 y)) + (x0l x0)                          (model.py:255-256)
__device__ __forceinline__ bf16_t mix_attn(const float* lam, float x, float x0, float y) {
  const float yb = rbf(y);
  const float t = rbf(rbf(lam[0] * x) + rbf(lam[2] * yb));
  return f2bf(t + rbf(lam[4] * x0));
}
//   x = (r1 x) + (p1 y)                                        (model.py:259-260)
__device__ __forceinline__ bf16_t mix_mlp(const float* lam, float x, float y) {
  return f2bf(rbf(lam[1] * x) + rbf(lam[3] * rbf(y)));
}
//   relu(y)^2                                                  (model.py:258)
__device__ __forceinline__ bf16_t relu2_bf(float y) {
  const float u = rbf(y);
  const float r = u > 0.f ? u : 0.f;
  return f2bf(r * r);
}
// mix_attn / mix_mlp of two bf16 pairs packed in words (y already bf16),
// each eager rounding done as one packed conversion of the pair.
__device__ __forceinline__ float lo_f(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ uint32_t mix_attn_pair(const float* lam, uint32_t x, uint32_t x0,
                                                  uint32_t y) {
  const uint32_t a = pack2(lam[0] * lo_f(x), lam[0] * hi_f(x));
  const uint32_t b = pack2(lam[2] * lo_f(y), lam[2] * hi_f(y));
  const uint32_t t = pack2(lo_f(a) + lo_f(b), hi_f(a) + hi_f(b));
  const uint32_t c = pack2(lam[4] * lo_f(x0), lam[4] * hi_f(x0));
  return pack2(lo_f(t) + lo_f(c), hi_f(t) + hi_f(c));
}
__device__ __forceinline__ uint32_t mix_mlp_pair(const float* lam, uint32_t x, uint32_t y) {
  const uint32_t a = pack2(lam[1] * lo_f(x), lam[1] * hi_f(x));
  const uint32_t b = pack2(lam[3] * lo_f(y), lam[3] * hi_f(y));
  return pack2(lo_f(a) + lo_f(b), hi_f(a) + hi_f(b));
}
// relu2_bf of two values as one packed word: bf16(max(y, 0)) equals
// max(bf16(y), 0) (rounding is monotone and keeps 0; NaN gives 0 on both
// sides), so the clamp goes first and each pair takes two packed conversions.
__device__ __forceinline__ uint32_t relu2_pair(float y0, float y1) {
  const uint32_t u = pack2(fmaxf(y0, 0.f), fmaxf(y1, 0.f));
  const float a = __uint_as_float(u << 16), b = __uint_as_float(u & 0xffff0000u);
  return pack2(a * a, b * b);
}
// Order-preserving 16-bit key of a bf16 value (greedy argmax).
__device__ __forceinline__ uint32_t zkey(bf16_t h) {
  return (h & 0x8000u) ? (uint32_t)(~h & 0xffffu) : (uint32_t)(h | 0x8000u);
}

// ---- tagged words ("LL" exchange) -------------------------------------------
// A 64-bit word carries 32 bits of data and a 32-bit tag, written with one
// relaxed device-scope store and read with device-scope loads: a reader that
// sees the tag it waits for has that writer's data of the same word.  Only
// single-location coherence is relied on -- no fence, no ordering between
// different words.
typedef unsigned long long u64;
constexpr unsigned LL_SPIN = 1u << 18;   // polls before a wait gives up

__device__ __forceinline__ void ll_store(u64* p, uint32_t v, uint32_t tag) {
  __hip_atomic_store(p, ((u64)tag << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u64 ll_load(const u64* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The waits below are inlined at every use: an out-of-line call opens with a
// wait for all of the caller's outstanding loads (prefetched weights, K/V
// rows), and through a generic pointer every poll becomes a flat load whose
// wait also covers LDS traffic.  Inline, the polls are global loads and the
// compiler waits for exactly the loads it needs.
//
// Wait until the word carries `tag` and return its data.  Bounded: after
// LL_SPIN polls, or once another wait has already given up (*err set), it
// sets *err and returns whatever it read last.
__device__ __forceinline__ uint32_t ll_wait(const u64* p, uint32_t tag, unsigned* err) {
  u64 v = ll_load(p);
  for (unsigned s = 1; (uint32_t)(v >> 32) != tag; ++s) {
    if ((s & 63u) == 0) {
      if (s >= LL_SPIN) {
        atomicOr(err, 1u);
        break;
      }
      if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
    }
    v = ll_load(p);
  }
  return (uint32_t)v;
}
// N words at once: v[j] holds a value already read from p[j] (ok[j] false:
// not a word of this thread, never waited for).  Re-reads the words that do
// not carry `tag` yet, all of them together, until every one does; bounded
// like ll_wait.
template <int N>
__device__ __forceinline__ void ll_settle(const u64* const (&p)[N], u64 (&v)[N], const bool (&ok)[N],
                                          uint32_t tag, unsigned* err) {
  for (unsigned s = 1;; ++s) {
    bool done = true;
#pragma unroll
    for (int j = 0; j < N; ++j) done = done && (!ok[j] || (uint32_t)(v[j] >> 32) == tag);
    if (done) return;
    if ((s & 63u) == 0) {
      if (s >= LL_SPIN) {
        atomicOr(err, 1u);
        return;
      }
      if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return;
    }
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (ok[j] && (uint32_t)(v[j] >> 32) != tag) v[j] = ll_load(p[j]);
  }
}
