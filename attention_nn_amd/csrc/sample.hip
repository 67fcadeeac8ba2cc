// Sampling of one token per row from bf16 z = lm_head logits before the
// softcap (sample.py:44-49):
//   greedy (temperature 0): argmax of z over the first Vs entries, lowest
//     index on ties (softcap is increasing, so this is the argmax of the
//     softcapped logits);
//   otherwise: zc = softcap(z) / temperature; kth = k-th largest zc; keep
//     every zc >= kth (ties included, as `where(z < kth, -1e9, z)`); draw
//     u ~ U[0,1) from Philox4x32-10 and return the first kept index whose
//     running sum of exp(zc - max) exceeds u * total.
// One work-group of 1024 threads per row; thread t holds the ordered 16-bit
// keys of entries [56 t, 56 t + 56) in registers, two per dword.  The k-th
// largest of the per-thread maxima, lb, bounds the k-th largest key from
// below (k <= the threads holding entries); wave 0 finds it by bisection over
// the maxima, 16 per lane, with wave reductions only.  Every key >= lb (at
// least k of them, and every kept one) is then copied to an LDS list, and if
// the list holds at most 1024 keys wave 0 bisects over it the same way for
// the k-th largest key.  A longer list (ties, flat logits, large k) falls
// back to a bisection over all keys with block-wide counts per round (packed
// saturating 16-bit arithmetic).  The weights use the hardware exp2 /
// reciprocal; only chunks holding a kept entry in some lane of the wave
// evaluate them.
#include <math.h>
#include "common.h"
#include "launch.h"

namespace ann {

constexpr int SMP_THREADS = 1024;
constexpr int SMP_CH = 7;              // 16-byte chunks (8 entries) per thread
constexpr int SMP_PER = SMP_CH * 8;    // entries per thread: Vs <= 57344
constexpr int SMP_CAP = 1024;          // candidate list: 16 keys per lane of one wave
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Two bf16 values of a dword -> their order-preserving 16-bit keys
// (negative: ~h, non-negative: h | 0x8000).
__device__ __forceinline__ uint32_t okey2(uint32_t w) {
  return w ^ (0x80008000u | (((w >> 15) & 0x00010001u) * 0x7fffu));
}
__device__ __forceinline__ float key2f(uint32_t k) {
  const uint32_t h = (k & 0x8000u) ? (k & 0x7fffu) : (~k & 0xffffu);
  return __uint_as_float(h << 16);
}
// Number of packed 16-bit keys >= t (t >= 1): sat(key - (t - 1)) > 0.
__device__ __forceinline__ uint32_t count_ge(const uint32_t* kk, uint32_t t) {
  const unsigned short t1 = (unsigned short)(t - 1);
  const u16x2 tm = {t1, t1}, one = {1, 1};
  u16x2 acc = {0, 0};
#pragma unroll
  for (int j = 0; j < SMP_PER / 2; ++j) {
    const u16x2 v = __builtin_bit_cast(u16x2, kk[j]);
    acc += __builtin_elementwise_min(__builtin_elementwise_sub_sat(v, tm), one);
  }
  return (uint32_t)acc.x + (uint32_t)acc.y;
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

// Wave reductions of the device library (fixed-order DPP row operations).
extern "C" __device__ unsigned long __ockl_wfred_max_u64(unsigned long);
extern "C" __device__ unsigned __ockl_wfred_max_u32(unsigned);
extern "C" __device__ unsigned __ockl_wfred_min_u32(unsigned);
extern "C" __device__ int __ockl_wfred_add_i32(int);

__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t* red) {
  v = __ockl_wfred_max_u64(v);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wv] = v;
  __syncthreads();
  uint64_t b = 0;
#pragma unroll
  for (int w = 0; w < SMP_THREADS / 64; ++w) b = red[w] > b ? red[w] : b;
  return b;
}

// Largest T in [lo, hi] with at least k of the wave's keys >= T (16 per lane
// as 8 packed pairs, 0 = no key; lo must satisfy it).  lo, hi and the counts
// are wave-uniform; every T tried is >= 1.
__device__ __forceinline__ uint32_t wave_kth(const uint32_t (&v)[8], uint32_t lo, uint32_t hi,
                                             uint32_t k) {
  const u16x2 one = {1, 1};
  while (lo < hi) {
    const uint32_t mid = (lo + hi + 1) >> 1;
    const unsigned short t1 = (unsigned short)(mid - 1);
    const u16x2 tm = {t1, t1};
    u16x2 acc = {0, 0};
#pragma unroll
    for (int j = 0; j < 8; ++j)
      acc += __builtin_elementwise_min(
          __builtin_elementwise_sub_sat(__builtin_bit_cast(u16x2, v[j]), tm), one);
    if ((uint32_t)__ockl_wfred_add_i32((int)((uint32_t)acc.x + (uint32_t)acc.y)) >= k) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// Block sum of per-wave counts (wc uniform within each wave); buf alternates
// between calls so that one barrier per call suffices.
__device__ __forceinline__ uint32_t block_sum_waves(uint32_t wc, uint32_t* buf) {
  if ((threadIdx.x & 63) == 0) buf[threadIdx.x >> 6] = wc;
  __syncthreads();
  uint32_t t = 0;
#pragma unroll
  for (int w = 0; w < SMP_THREADS / 64; ++w) t += buf[w];
  return t;
}

// The draw for one row from the ordered 16-bit keys of this thread's entries
// [base, base + nvalid), base = 56 tid (key 0 past the valid entries): the
// whole-row sampler of k_sample, shared with k_sample_cand's fallback.
__device__ __forceinline__ void sample_keys_row(uint32_t (&kk)[SMP_PER / 2], int Vs, int row,
                                                float temperature, int top_k, uint64_t seed,
                                                uint64_t step, int32_t pos0,
                                                unsigned long long* __restrict__ steps,
                                                int32_t* __restrict__ out_tok,
                                                int32_t* __restrict__ pos, int pos_adv) {
  __shared__ uint32_t s_cnt[2][SMP_THREADS / 64];
  __shared__ uint64_t s_red[SMP_THREADS / 64];
  __shared__ uint32_t s_mm[2][SMP_THREADS / 64];
  __shared__ float s_wsum[SMP_THREADS / 64];
  __shared__ uint32_t s_misc[2];
  __shared__ __attribute__((aligned(16))) unsigned short s_lmax[SMP_THREADS];
  __shared__ __attribute__((aligned(16))) unsigned short s_list[SMP_CAP];
  __shared__ uint32_t s_sel[2];   // [0] bound / threshold broadcast, [1] list length
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int base = tid * SMP_PER;
  const int nvalid = max(0, min(SMP_PER, Vs - base));
  uint32_t lmax = 0;
  int lidx = 0;
#pragma unroll
  for (int j = 0; j < SMP_PER / 2; ++j) {
    const uint32_t lo = kk[j] & 0xffffu, hi = kk[j] >> 16;
    if (lo > lmax) { lmax = lo; lidx = 2 * j; }
    if (hi > lmax) { lmax = hi; lidx = 2 * j + 1; }
  }

  if (temperature == 0.f) {   // greedy: maximal key, lowest index on ties
    uint64_t best = ((uint64_t)lmax << 32) | (uint64_t)(0xffffffffu - (uint32_t)(base + lidx));
    best = block_max_u64(best, s_red);
    if (tid == 0) {
      out_tok[row] = (int32_t)(0xffffffffu - (uint32_t)(best & 0xffffffffu));
      if (pos) pos[row] = pos0 + pos_adv;
    }
    return;
  }
  // maximum key, and the smallest per-thread maximum over threads holding
  // entries (a lower bound of the k-th largest key when top_k <= those threads)
  {
    const uint32_t wmax = __ockl_wfred_max_u32(lmax);
    const uint32_t wmin = __ockl_wfred_min_u32(nvalid > 0 ? lmax : 0xffffffffu);
    if (lane == 0) {
      s_mm[0][wv] = wmax;
      s_mm[1][wv] = wmin;
    }
    s_lmax[tid] = (unsigned short)lmax;
    if (tid == 0) s_sel[1] = 0u;
  }
  __syncthreads();
  uint32_t kmax = 0, lmin = 0xffffffffu;
#pragma unroll
  for (int w = 0; w < SMP_THREADS / 64; ++w) {
    kmax = s_mm[0][w] > kmax ? s_mm[0][w] : kmax;
    lmin = s_mm[1][w] < lmin ? s_mm[1][w] : lmin;
  }
  const int holders = (Vs + SMP_PER - 1) / SMP_PER;   // threads with entries

  // ---- k-th largest key: largest T with count(key >= T) >= top_k
  uint32_t thr_key = 0;
  const bool use_thr = top_k > 0 && top_k < Vs;
  if (use_thr) {
    uint32_t lo = 0, hi = kmax;
    bool found = false;
    if (top_k <= holders) {
      // lower bound: the top_k-th largest per-thread maximum (top_k threads
      // each hold a key >= it), searched above the smallest maximum, which
      // every holder reaches (threads without entries have maximum 0)
      if (wv == 0) {
        uint32_t v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = ((const uint32_t*)s_lmax)[j * 64 + lane];
        const uint32_t lb = wave_kth(v, lmin, kmax, (uint32_t)top_k);
        if (lane == 0) s_sel[0] = lb;
      }
      __syncthreads();
      lo = s_sel[0];
      if (lo > 0u) {
        // candidates: every key >= lo, placed by a wave scan of the counts
        const uint32_t cnt = count_ge(kk, lo);
        uint32_t incl = cnt;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const uint32_t v = __shfl_up(incl, o, 64);
          if (lane >= o) incl += v;
        }
        uint32_t wb = 0;
        if (lane == 63) wb = atomicAdd(&s_sel[1], incl);
        wb = __shfl(wb, 63, 64);
        if (cnt) {
          uint32_t p = wb + incl - cnt;
#pragma unroll
          for (int j = 0; j < SMP_PER / 2; ++j) {
            const uint32_t a = kk[j] & 0xffffu, b = kk[j] >> 16;
            if (a >= lo) { if (p < (uint32_t)SMP_CAP) s_list[p] = (unsigned short)a; ++p; }
            if (b >= lo) { if (p < (uint32_t)SMP_CAP) s_list[p] = (unsigned short)b; ++p; }
          }
        }
        __syncthreads();
        const uint32_t n = s_sel[1];   // >= top_k
        if (n <= (uint32_t)SMP_CAP) {
          // every key >= the k-th largest is listed: the list's k-th largest
          if (wv == 0) {
            uint32_t v[8];   // list entries 2i, 2i + 1; entries >= n read as 0
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              const uint32_t i = (uint32_t)(j * 64 + lane);
              const uint32_t w = ((const uint32_t*)s_list)[i];
              v[j] = (2 * i < n ? (w & 0xffffu) : 0u) | (2 * i + 1 < n ? (w & 0xffff0000u) : 0u);
            }
            const uint32_t t = wave_kth(v, lo, hi, (uint32_t)top_k);
            if (lane == 0) s_sel[0] = t;
          }
          __syncthreads();
          thr_key = s_sel[0];
          found = true;
        }
      }
    }
    if (!found) {
      int round = 0;
      while (lo < hi) {
        const uint32_t mid = (lo + hi + 1) >> 1;
        const uint32_t c = (uint32_t)__ockl_wfred_add_i32((int)count_ge(kk, mid));
        const uint32_t tot = block_sum_waves(c, s_cnt[round++ & 1]);
        if (tot >= (uint32_t)top_k) lo = mid;
        else hi = mid - 1;
      }
      thr_key = lo;
    }
  }

  // ---- kept set = keys >= tk.  softcap / temperature is non-decreasing in
  // z, so zc >= zc(thr_key) is key >= thr_key unless keys below thr_key
  // round to the same zc (saturated softcap): then tk is the smallest such
  // key, found by bisection on the IEEE softcap.
  const float tmp = temperature;
  uint32_t tk = thr_key > 1u ? thr_key : 1u;
  if (use_thr && thr_key > 1u) {
    const float zthr = softcap(key2f(thr_key)) / tmp;
    if (softcap(key2f(thr_key - 1)) / tmp >= zthr) {
      uint32_t a = 1, b = thr_key - 1;   // smallest key in [1, thr_key-1] with f >= zthr
      while (a < b) {
        const uint32_t mid = (a + b) >> 1;
        if (softcap(key2f(mid)) / tmp >= zthr) b = mid;
        else a = mid + 1;
      }
      tk = a;
    }
  }

  // ---- weights exp((zc - zc_max) / T) of kept entries, per 8-entry chunk
  const float c2 = 1.4426950408889634f / tmp;   // log2(e) / T
  const float scmax = softcap_fast(key2f(kmax));
  auto wt = [&](uint32_t k) -> float {
    return __builtin_amdgcn_exp2f((softcap_fast(key2f(k)) - scmax) * c2);
  };
  float csum[SMP_CH];
  float local = 0.f;
  int lastk = -1;
#pragma unroll
  for (int c = 0; c < SMP_CH; ++c) {
    float s = 0.f;
#pragma unroll
    for (int j = 4 * c; j < 4 * c + 4; ++j) {
      const uint32_t lo = kk[j] & 0xffffu, hi = kk[j] >> 16;
      const bool klo = lo >= tk, khi = hi >= tk;
      if (__ballot(klo || khi)) {
        if (klo) { s += wt(lo); lastk = base + 2 * j; }
        if (khi) { s += wt(hi); lastk = base + 2 * j + 1; }
      }
    }
    csum[c] = s;
    local += s;
  }

  // ---- block exclusive scan of the per-thread sums (fixed order)
  float incl = local;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float v = __shfl_up(incl, o, 64);
    if (lane >= o) incl += v;
  }
  if (lane == 63) s_wsum[wv] = incl;
  if (tid == 0) { s_misc[0] = 0xffffffffu; s_misc[1] = 0u; }
  __syncthreads();
  float wbase = 0.f, total = 0.f;
#pragma unroll
  for (int w = 0; w < SMP_THREADS / 64; ++w) {
    if (w < wv) wbase += s_wsum[w];
    total += s_wsum[w];
  }
  const float before = wbase + incl - local;
  const uint32_t rw = philox_x((uint32_t)step, (uint32_t)row, (uint32_t)(step >> 32), 0u,
                               (uint32_t)seed, (uint32_t)(seed >> 32));
  const float target = (float)(rw >> 8) * (1.0f / 16777216.0f) * total;

  // ---- the thread whose interval holds the target walks its entries
  if (local > 0.f && target >= before && target < before + local) {
    float run = before;
    int pick = -1;
#pragma unroll
    for (int c = 0; c < SMP_CH; ++c) {
      if (pick < 0 && target < run + csum[c]) {
        float s = 0.f;   // same additions as csum[c]: reaches run + csum[c]
#pragma unroll
        for (int j = 4 * c; j < 4 * c + 4; ++j) {
          const uint32_t lo = kk[j] & 0xffffu, hi = kk[j] >> 16;
          if (lo >= tk) { s += wt(lo); if (pick < 0 && target < run + s) pick = base + 2 * j; }
          if (hi >= tk) { s += wt(hi); if (pick < 0 && target < run + s) pick = base + 2 * j + 1; }
        }
      }
      run += csum[c];
    }
    if (pick < 0) pick = lastk;
    atomicMin(&s_misc[0], (uint32_t)pick);
  }
  if (lastk >= 0) atomicMax(&s_misc[1], (uint32_t)lastk);
  __syncthreads();
  if (tid == 0) {
    // rounding can leave the target at/after every interval: last kept entry
    const uint32_t pick = s_misc[0] != 0xffffffffu ? s_misc[0] : s_misc[1];
    out_tok[row] = (int32_t)pick;
    if (pos) pos[row] = pos0 + pos_adv;
    steps[row] = step + 1;
  }
}

__global__ __launch_bounds__(SMP_THREADS) void k_sample(const bf16_t* __restrict__ zall, int ldz,
                                                        int Vs, const SampParams* __restrict__ sp,
                                                        unsigned long long* __restrict__ steps,
                                                        int32_t* __restrict__ out_tok,
                                                        int32_t* __restrict__ pos, int pos_adv) {
  const float temperature = sp->temperature;
  const int top_k = sp->top_k;
  const uint64_t seed = sp->seed;
  const int row = blockIdx.x, tid = threadIdx.x;
  // this row's position and step, read now rather than behind the last barrier
  const int32_t pos0 = pos ? pos[row] : 0;
  const uint64_t step = steps[row];
  const bf16_t* z = zall + (size_t)row * ldz;
  const int base = tid * SMP_PER;
  const int nvalid = max(0, min(SMP_PER, Vs - base));

  // ---- keys of this thread's entries; entries >= Vs get key 0.  A chunk
  // that starts below Vs lies inside the row's padded width (ldz >= Vs
  // rounded up to 8, checked on the host).
  uint32_t kk[SMP_PER / 2];
#pragma unroll
  for (int c = 0; c < SMP_CH; ++c) {
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (c * 8 < nvalid) v = *(const uint4*)(z + base + c * 8);
    kk[4 * c + 0] = okey2(v.x);
    kk[4 * c + 1] = okey2(v.y);
    kk[4 * c + 2] = okey2(v.z);
    kk[4 * c + 3] = okey2(v.w);
  }
  if (nvalid < SMP_PER) {
#pragma unroll
    for (int j = 0; j < SMP_PER / 2; ++j)
      kk[j] &= (2 * j < nvalid ? 0xffffu : 0u) | (2 * j + 1 < nvalid ? 0xffff0000u : 0u);
  }
  sample_keys_row(kk, Vs, row, temperature, top_k, seed, step, pos0, steps, out_tok, pos,
                  pos_adv);
}

// ---- draws from the lm_head's top-k candidates -------------------------------
//
// Each tile t -- a 128-column tile of the lm_head GEMM (EPI_TOPK), or one
// work-group's row slice of the persistent step -- left, per row, its TK_M
// largest words (key << 16 | 0xffff - n, largest first) and its next largest
// word r_t.  Thread t holds tile t's candidates.  The k-th largest candidate
// key T is found like k_sample's threshold: a lower bound lb from the tile
// maxima, then the keys above it listed and bisected.  If every tile's next
// key r_t lies below the kept threshold tk (<= T), every key >= tk is a
// candidate: the k-th largest key of the row is T (any larger k-th key would
// have k candidates above T) and the kept set is the candidates >= tk.  When
// the list holds at most 64 keys and that is already settled at lb, wave 0
// finishes alone (ballot-count bisection, a bitonic sort of the kept items
// into column order across the lanes, a wave scan); otherwise the block
// draws.  Where the candidates cannot settle it, the row is sampled whole:
// from z when the producer stored it (the persistent step), else the tiles
// with r_t >= tk (all tiles when T could not be formed) are recomputed into
// an LDS row of keys -- the others contribute their candidates, the rest of
// their keys lying below tk and below any threshold the full row can give --
// and k_sample's whole-row draw runs on that row.  The recomputation repeats
// the lm_head GEMM's accumulation for the row: one v_mfma_f32_16x16x32_bf16
// per 32-wide k step in k order, W as the first operand, the row as column 0
// of the second, so z is bit-identical.  (Measured: the whole draw in one
// wave, counting over 64 words per lane, took 14-15 us at 64 rows against
// 10 us for the block form then -- one wave issues at a quarter of the CU's
// VALU rate; the single-wave finish above works on one key per lane.)

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

// ascending compare-exchange
__device__ __forceinline__ void cas(uint32_t& a, uint32_t& b) {
  const uint32_t lo = min(a, b), hi = max(a, b);
  a = lo;
  b = hi;
}

__global__ __launch_bounds__(SMP_THREADS) void k_sample_cand(
    const uint32_t* __restrict__ cand, const uint32_t* __restrict__ cand_r, int nt, int holders,
    int Vs, const bf16_t* __restrict__ zfb, const bf16_t* __restrict__ A, int lda,
    const bf16_t* __restrict__ W, int N, int K,
    const SampParams* __restrict__ sp, unsigned long long* __restrict__ steps,
    int32_t* __restrict__ out_tok, int32_t* __restrict__ pos, int pos_adv,
    unsigned* __restrict__ verify) {
  extern __shared__ __attribute__((aligned(16))) unsigned short s_row[];   // nt * 128 keys
  __shared__ uint32_t s_mx[3][SMP_THREADS / 64];
  __shared__ uint32_t s_cnt[2][SMP_THREADS / 64];
  __shared__ float s_wsum[SMP_THREADS / 64];
  __shared__ uint32_t s_misc[2];
  __shared__ __attribute__((aligned(16))) unsigned short s_lmax[SMP_THREADS];
  __shared__ uint32_t s_item[SMP_CAP];   // listed candidates: n << 16 | key
  __shared__ uint32_t s_sel[3];   // [0] bound / threshold, [1] list length, [2] see below
  __shared__ uint32_t s_nf;
  __shared__ unsigned short s_flag[SMP_THREADS];
  const float temperature = sp->temperature;
  const int top_k = sp->top_k;
  const uint64_t seed = sp->seed;
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int32_t pos0 = pos ? pos[row] : 0;
  const uint64_t step = steps[row];
  uint32_t cw[TK_M], rw = 0u;   // holders: the tiles with valid columns
  if (tid < holders) {
    const uint4* src = (const uint4*)(cand + ((size_t)row * nt + tid) * TK_M);
    const uint4 a = src[0], b = src[1];
    cw[0] = a.x; cw[1] = a.y; cw[2] = a.z; cw[3] = a.w;
    cw[4] = b.x; cw[5] = b.y; cw[6] = b.z; cw[7] = b.w;
    rw = cand_r[(size_t)row * nt + tid];
  } else {
#pragma unroll
    for (int e = 0; e < TK_M; ++e) cw[e] = 0u;
  }
  const uint32_t wtop = cw[0];   // the tile's largest word
  const uint32_t lmax = wtop >> 16;
  // block maxima: the top word (greedy), the top key, the largest non-candidate
  // key; the smallest tile maximum over the holders
  {
    const uint32_t a = __ockl_wfred_max_u32(wtop);
    const uint32_t b = __ockl_wfred_max_u32(rw >> 16);
    const uint32_t c = __ockl_wfred_min_u32(tid < holders ? lmax : 0xffffffffu);
    if (lane == 0) {
      s_mx[0][wv] = a;
      s_mx[1][wv] = b;
      s_mx[2][wv] = c;
    }
    s_lmax[tid] = (unsigned short)lmax;
    if (tid == 0) { s_sel[1] = 0u; s_nf = 0u; }
  }
  __syncthreads();
  uint32_t gtop = 0u, rmax = 0u, lmin = 0xffffffffu;
#pragma unroll
  for (int w = 0; w < SMP_THREADS / 64; ++w) {
    gtop = max(gtop, s_mx[0][w]);
    rmax = max(rmax, s_mx[1][w]);
    lmin = min(lmin, s_mx[2][w]);
  }
  if (temperature == 0.f) {   // greedy: the tiles' largest words hold the row's
    if (tid == 0) {
      out_tok[row] = (int32_t)(0xffffu - (gtop & 0xffffu));
      if (pos) pos[row] = pos0 + pos_adv;
    }
    return;
  }
  const uint32_t kmax = gtop >> 16;

  // ---- k-th largest candidate key T (as in sample_keys_row)
  bool fast = top_k > 0 && top_k < Vs && top_k <= holders;
  uint32_t thr = 0u;
  if (fast) {
    if (wv == 0) {   // (a ballot count per 64 maxima measured slower: 2.6 against 1.8 us)
      uint32_t v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = ((const uint32_t*)s_lmax)[j * 64 + lane];
      const uint32_t lb = wave_kth(v, lmin, kmax, (uint32_t)top_k);
      if (lane == 0) {
        s_sel[0] = lb;
        // 1: no key below lb rounds to the softcapped value of lb (tk >= lb)
        s_sel[2] = softcap(key2f(lb - 1)) / temperature < softcap(key2f(lb)) / temperature;
      }
    }
    __syncthreads();
    const uint32_t lo = s_sel[0];
    uint32_t cnt = 0;
#pragma unroll
    for (int e = 0; e < TK_M; ++e) cnt += (cw[e] >> 16) >= lo ? 1u : 0u;
    uint32_t incl = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t v = __shfl_up(incl, o, 64);
      if (lane >= o) incl += v;
    }
    uint32_t wb = 0;
    if (lane == 63) wb = atomicAdd(&s_sel[1], incl);
    wb = __shfl(wb, 63, 64);
    if (cnt) {
      uint32_t p = wb + incl - cnt;
#pragma unroll
      for (int e = 0; e < TK_M; ++e) {
        const uint32_t k = cw[e] >> 16;
        if (k >= lo) {
          if (p < (uint32_t)SMP_CAP) s_item[p] = ((0xffffu - (cw[e] & 0xffffu)) << 16) | k;
          ++p;
        }
      }
    }
    __syncthreads();
    const uint32_t n = s_sel[1];   // >= top_k
    // At most 64 listed keys, every non-candidate key below lo, and no key
    // below lo rounding to the softcapped value of lo (so tk >= lo and the
    // kept set lies in the list): wave 0 finishes alone, one item per lane.
    if (n <= 64u && rmax < lo && !verify && s_sel[2]) {
      if (wv != 0) return;
      const uint32_t it = lane < (int)n ? s_item[lane] : 0u;
      const uint32_t key = it & 0xffffu;
      uint32_t a = lo, b = kmax;   // T: the top_k-th largest listed key
      while (a < b) {
        const uint32_t mid = (a + b + 1) >> 1;
        if ((uint32_t)__builtin_popcountll(__ballot(key >= mid)) >= (uint32_t)top_k) a = mid;
        else b = mid - 1;
      }
      const uint32_t t1 = a;
      uint32_t tq = t1;   // tk in [lo, T] (the softcap saturation rule)
      const float zthr = softcap(key2f(t1)) / temperature;
      if (t1 > lo && softcap(key2f(t1 - 1)) / temperature >= zthr) {
        uint32_t c = lo, e = t1 - 1;
        while (c < e) {
          const uint32_t mid = (c + e) >> 1;
          if (softcap(key2f(mid)) / temperature >= zthr) e = mid;
          else c = mid + 1;
        }
        tq = c;
      }
      // kept items in column order: a bitonic sort of (n << 16 | key) over
      // the lanes, dropped ones ~0 (last)
      uint32_t sv = key >= tq && lane < (int)n ? it : 0xffffffffu;
#pragma unroll
      for (int kk = 2; kk <= 64; kk <<= 1)
#pragma unroll
        for (int jj = kk >> 1; jj > 0; jj >>= 1) {
          const uint32_t o = (uint32_t)__shfl_xor((int)sv, jj, 64);
          const bool asc = (lane & kk) == 0, low = (lane & jj) == 0;
          sv = (asc == low) ? min(sv, o) : max(sv, o);
        }
      const int nk = __builtin_popcountll(__ballot(sv != 0xffffffffu));
      const float c2 = 1.4426950408889634f / temperature;
      const float scmax = softcap_fast(key2f(kmax));
      const float w = lane < nk ? __builtin_amdgcn_exp2f(
                                      (softcap_fast(key2f(sv & 0xffffu)) - scmax) * c2)
                                : 0.f;
      float incl = w;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const float x = __shfl_up(incl, o, 64);
        if (lane >= o) incl += x;
      }
      const float total = __shfl(incl, 63, 64);
      const uint32_t rwd = philox_x((uint32_t)step, (uint32_t)row, (uint32_t)(step >> 32), 0u,
                                    (uint32_t)seed, (uint32_t)(seed >> 32));
      const float target = (float)(rwd >> 8) * (1.0f / 16777216.0f) * total;
      // the first item whose running sum exceeds the target; rounding can
      // leave the target at or past the last: then the last kept item
      const uint64_t hit = __ballot(lane < nk && target < incl);
      const int src = hit ? __builtin_ctzll(hit) : nk - 1;
      const uint32_t tok = (uint32_t)__shfl((int)sv, src, 64) >> 16;
      if (lane == 0) {
        out_tok[row] = (int32_t)tok;
        if (pos) pos[row] = pos0 + pos_adv;
        steps[row] = step + 1;
      }
      return;
    }
    if (n <= (uint32_t)SMP_CAP) {
      if (wv == 0) {   // keys of items 2i and 2i + 1, i = 64 j + lane
        uint32_t v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t i = (uint32_t)(j * 64 + lane);
          const uint32_t k0 = 2 * i < n ? (s_item[2 * i] & 0xffffu) : 0u;
          const uint32_t k1 = 2 * i + 1 < n ? (s_item[2 * i + 1] & 0xffffu) : 0u;
          v[j] = k0 | (k1 << 16);
        }
        const uint32_t t = wave_kth(v, lo, kmax, (uint32_t)top_k);
        if (lane == 0) s_sel[0] = t;
      }
      __syncthreads();
      thr = s_sel[0];
    } else {
      uint32_t a = lo, b = kmax;
      int round = 0;
      while (a < b) {
        const uint32_t mid = (a + b + 1) >> 1;
        uint32_t c = 0;
#pragma unroll
        for (int e = 0; e < TK_M; ++e) c += (cw[e] >> 16) >= mid ? 1u : 0u;
        c = (uint32_t)__ockl_wfred_add_i32((int)c);
        const uint32_t tot = block_sum_waves(c, s_cnt[round++ & 1]);
        if (tot >= (uint32_t)top_k) a = mid;
        else b = mid - 1;
      }
      thr = a;
    }
  }
  // kept set = keys >= tk (the softcap saturation rule of sample_keys_row)
  const float tmp = temperature;
  uint32_t tk = thr > 1u ? thr : 1u;
  if (fast && thr > 1u) {
    const float zthr = softcap(key2f(thr)) / tmp;
    if (softcap(key2f(thr - 1)) / tmp >= zthr) {
      uint32_t a = 1, b = thr - 1;
      while (a < b) {
        const uint32_t mid = (a + b) >> 1;
        if (softcap(key2f(mid)) / tmp >= zthr) b = mid;
        else a = mid + 1;
      }
      tk = a;
    }
  }
  // verify (a check of the recomputation): every tile with more than TK_M
  // valid columns is recomputed and its top TK_M + 1 words compared with the
  // GEMM's; a difference sets bit 1 of *verify
  fast = fast && rmax < tk && !verify;

  if (fast) {
    // ---- kept candidates of this thread in column order: (n << 16 | key),
    // dropped ones ~0
    uint32_t it[TK_M];
#pragma unroll
    for (int e = 0; e < TK_M; ++e)
      it[e] = (cw[e] >> 16) >= tk ? ((0xffffu - (cw[e] & 0xffffu)) << 16) | (cw[e] >> 16)
                                  : 0xffffffffu;
    // Batcher's odd-even merge sort of 8
    cas(it[0], it[1]); cas(it[2], it[3]); cas(it[4], it[5]); cas(it[6], it[7]);
    cas(it[0], it[2]); cas(it[1], it[3]); cas(it[4], it[6]); cas(it[5], it[7]);
    cas(it[1], it[2]); cas(it[5], it[6]);
    cas(it[0], it[4]); cas(it[1], it[5]); cas(it[2], it[6]); cas(it[3], it[7]);
    cas(it[2], it[4]); cas(it[3], it[5]);
    cas(it[1], it[2]); cas(it[3], it[4]); cas(it[5], it[6]);
    const float c2 = 1.4426950408889634f / tmp;
    const float scmax = softcap_fast(key2f(kmax));
    auto wt = [&](uint32_t k) -> float {
      return __builtin_amdgcn_exp2f((softcap_fast(key2f(k)) - scmax) * c2);
    };
    float local = 0.f;
    int lastk = -1;
#pragma unroll
    for (int e = 0; e < TK_M; ++e)
      if (it[e] != 0xffffffffu) {
        local += wt(it[e] & 0xffffu);
        lastk = (int)(it[e] >> 16);
      }
    float incl = local;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float v = __shfl_up(incl, o, 64);
      if (lane >= o) incl += v;
    }
    if (lane == 63) s_wsum[wv] = incl;
    if (tid == 0) { s_misc[0] = 0xffffffffu; s_misc[1] = 0u; }
    __syncthreads();
    float wbase = 0.f, total = 0.f;
#pragma unroll
    for (int w = 0; w < SMP_THREADS / 64; ++w) {
      if (w < wv) wbase += s_wsum[w];
      total += s_wsum[w];
    }
    const float before = wbase + incl - local;
    const uint32_t rwd = philox_x((uint32_t)step, (uint32_t)row, (uint32_t)(step >> 32), 0u,
                                  (uint32_t)seed, (uint32_t)(seed >> 32));
    const float target = (float)(rwd >> 8) * (1.0f / 16777216.0f) * total;
    if (local > 0.f && target >= before && target < before + local) {
      float run = before;
      int pick = -1;
#pragma unroll
      for (int e = 0; e < TK_M; ++e)
        if (it[e] != 0xffffffffu) {   // same additions as local
          run += wt(it[e] & 0xffffu);
          if (pick < 0 && target < run) pick = (int)(it[e] >> 16);
        }
      if (pick < 0) pick = lastk;
      atomicMin(&s_misc[0], (uint32_t)pick);
    }
    if (lastk >= 0) atomicMax(&s_misc[1], (uint32_t)lastk);
    __syncthreads();
    if (tid == 0) {
      const uint32_t pick = s_misc[0] != 0xffffffffu ? s_misc[0] : s_misc[1];
      out_tok[row] = (int32_t)pick;
      if (pos) pos[row] = pos0 + pos_adv;
      steps[row] = step + 1;
    }
    return;
  }

  if (zfb) {   // the producer also stored z: k_sample's draw on it
    const bf16_t* z = zfb + (size_t)row * N;
    const int base = tid * SMP_PER;
    const int nvalid = max(0, min(SMP_PER, Vs - base));
    uint32_t kk[SMP_PER / 2];
#pragma unroll
    for (int c = 0; c < SMP_CH; ++c) {
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (c * 8 < nvalid) v = *(const uint4*)(z + base + c * 8);
      kk[4 * c + 0] = okey2(v.x);
      kk[4 * c + 1] = okey2(v.y);
      kk[4 * c + 2] = okey2(v.z);
      kk[4 * c + 3] = okey2(v.w);
    }
    if (nvalid < SMP_PER) {
#pragma unroll
      for (int j = 0; j < SMP_PER / 2; ++j)
        kk[j] &= (2 * j < nvalid ? 0xffffu : 0u) | (2 * j + 1 < nvalid ? 0xffff0000u : 0u);
    }
    sample_keys_row(kk, Vs, row, temperature, top_k, seed, step, pos0, steps, out_tok, pos,
                    pos_adv);
    return;
  }

  // ---- whole row in LDS: candidates of the tiles whose other keys lie below
  // fl, recomputed keys of the rest
  const uint32_t fl = thr > 0u && !verify ? tk : 1u;
  const int nk8 = nt * 16;   // 16-byte chunks of the row
  for (int i = tid; i < nk8; i += SMP_THREADS) ((uint4*)s_row)[i] = make_uint4(0u, 0u, 0u, 0u);
  __syncthreads();
  if (tid < holders) {
    if ((rw >> 16) >= fl) {
      s_flag[atomicAdd(&s_nf, 1u)] = (unsigned short)tid;
    } else {
#pragma unroll
      for (int e = 0; e < TK_M; ++e)
        if (cw[e]) s_row[0xffffu - (cw[e] & 0xffffu)] = (unsigned short)(cw[e] >> 16);
    }
  }
  __syncthreads();
  const int nf = (int)s_nf;
  const bf16_t* arow = A + (size_t)row * lda;
  const bf16x8_t zero8 = {};
  for (int f = wv; f < nf; f += SMP_THREADS / 64) {
    const int t = s_flag[f];
    floatx4_t acc[8];
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) acc[nb] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
    const bf16_t* wr[8];
#pragma unroll
    for (int nb = 0; nb < 8; ++nb)
      wr[nb] = W + (size_t)min(t * 128 + nb * 16 + (lane & 15), N - 1) * K + (lane >> 4) * 8;
    for (int k0 = 0; k0 < K; k0 += 32) {
      const bf16x8_t a =
          (lane & 15) == 0 ? *(const bf16x8_t*)(arow + k0 + (lane >> 4) * 8) : zero8;
#pragma unroll
      for (int nb = 0; nb < 8; ++nb)
        acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const bf16x8_t*)(wr[nb] + k0), a,
                                                          acc[nb], 0, 0, 0);
    }
    // lane (lane & 15) == 0 holds rows n = 4 (lane >> 4) + r of each block
    if ((lane & 15) == 0) {
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) {
        const int n = t * 128 + nb * 16 + (lane >> 4) * 4;
        uint32_t kq[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) kq[r] = n + r < Vs ? zkey(f2bf(acc[nb][r])) : 0u;
        *(uint2*)(s_row + n) = make_uint2(kq[0] | (kq[1] << 16), kq[2] | (kq[3] << 16));
      }
    }
  }
  __syncthreads();
  if (verify && tid < holders && (rw >> 16) >= fl) {
    // the recomputed tile's TK_M + 1 largest words are the GEMM's
    bool ok = s_row[0xffffu - (rw & 0xffffu)] == (rw >> 16);
#pragma unroll
    for (int e = 0; e < TK_M; ++e)
      ok = ok && cw[e] != 0u && s_row[0xffffu - (cw[e] & 0xffffu)] == (cw[e] >> 16);
    uint32_t above = 0;
    for (int j = 0; j < 128; ++j) {
      const int n = tid * 128 + j;
      if (n < Vs) above += (((uint32_t)s_row[n] << 16) | (0xffffu - (uint32_t)n)) > rw ? 1u : 0u;
    }
    if (!ok || above != (uint32_t)TK_M) atomicOr(verify, 2u);
  }
  const int base = tid * SMP_PER;
  const int nvalid = max(0, min(SMP_PER, Vs - base));
  uint32_t kk[SMP_PER / 2];
#pragma unroll
  for (int c = 0; c < SMP_CH; ++c) {
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (c * 8 < nvalid) v = *(const uint4*)(s_row + base + c * 8);
    kk[4 * c + 0] = v.x;
    kk[4 * c + 1] = v.y;
    kk[4 * c + 2] = v.z;
    kk[4 * c + 3] = v.w;
  }
  sample_keys_row(kk, Vs, row, temperature, top_k, seed, step, pos0, steps, out_tok, pos,
                  pos_adv);
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
  if (Vs < 1 || Vs > SMP_THREADS * SMP_PER || ldz % 8 || ((Vs + 7) & ~7) > ldz)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_sample, dim3(B), dim3(SMP_THREADS), 0, st, z, ldz, Vs, sp, steps, out_tok,
                     pos, pos_adv);
  return hipGetLastError();
}

hipError_t sample_prepare() {
  static const hipError_t attr = hipFuncSetAttribute(
      (const void*)k_sample_cand, hipFuncAttributeMaxDynamicSharedMemorySize, 128 * 1024);
  return attr;
}

hipError_t sample_cand(const uint32_t* cand, const uint32_t* cand_r, int nt, int holders, int B,
                       int Vs, const bf16_t* z, const bf16_t* A, int lda, const bf16_t* W, int N,
                       int K, const SampParams* sp, unsigned long long* steps, int32_t* out_tok,
                       int32_t* pos, int pos_adv, unsigned* verify, hipStream_t st) {
  if (Vs < 1 || Vs > N || N > 65536 || holders < 1 || holders > nt || nt > SMP_THREADS ||
      Vs > SMP_THREADS * SMP_PER || ((uintptr_t)cand & 15))
    return hipErrorInvalidValue;
  size_t lds = 0;
  if (z) {   // fallback from z (B, N)
    if (N % 8 || ((uintptr_t)z & 15) || verify) return hipErrorInvalidValue;
  } else {   // fallback recomputing the GEMM's 128-column tiles
    if (nt != (N + 127) / 128 || holders != (Vs + 127) / 128 || K % 32 || K < 32 || lda % 8 ||
        ((uintptr_t)A & 15) || ((uintptr_t)W & 15))
      return hipErrorInvalidValue;
    lds = (size_t)nt * 128 * 2;
    const hipError_t attr = sample_prepare();
    if (attr != hipSuccess) return attr;
    if (lds > 128 * 1024) return hipErrorInvalidValue;
  }
  hipLaunchKernelGGL(k_sample_cand, dim3(B), dim3(SMP_THREADS), lds, st, cand, cand_r, nt,
                     holders, Vs, z, A, lda, W, N, K, sp, steps, out_tok, pos, pos_adv, verify);
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
