// Prefill attention of B x T query rows against the bf16 KV cache
// (model.py:248-254): keep key j for query position p iff j <= p and, on the
// windowed layers, p - j < window.  Scores 0.1 * q.k in fp32, softmax in fp32,
// P.V accumulated in fp32, output rounded once to bf16.
#include <math.h>
#include "common.h"
#include "launch.h"

namespace ann {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

// ---- prefill: MFMA flash attention ------------------------------------------
//
// Grid (ceil(T/128), H, B), 512 threads: 8 waves x 16 queries.  Per 64-key
// tile, K and V are staged row-major in LDS (16-byte stores) and the next tile
// is fetched into registers meanwhile.  Each wave computes S^T = K Q^T with
// v_mfma_f32_16x16x32_bf16 (keys as rows, its 16 queries as columns) so the
// score fragments are already in the B-operand layout of O^T = V^T P^T:
// k index g*8 + e of a lane maps to key 32i + 4g + e (e < 4) and
// 32i + 16 + 4g + e - 4 (e >= 4).  The V^T A-operand comes straight from the
// row-major V tile through ds_read_b64_tr_b16: within each 16-lane group g,
// output lane m, element e is element (m & 3) of the 4-element row addressed
// by lane 4e + (m >> 2); lane i therefore points at key 32i + 4g + (i >> 2)
// (+16 for the second half), dims 16 db + 4 (i & 3), and lane m receives
// V[32i + 4g + e][16 db + m] for e = 0..3.  P enters the MFMA as bf16 hi +
// bf16 lo (two MFMAs), keeping P.V at ~2^-17 relative accuracy.  Softmax:
// fixed shift, as in the decode kernel (|score| <= scale * Dh).  Key tiles
// entirely outside the causal window of the query block are never visited; a
// wave skips the tiles outside its own 16 queries' window and evaluates the
// mask only on tiles that cross the diagonal or the window edge.

typedef short ap_v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) ap_v4i16 ap_lds_v4i16;

template <int DH>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void k_attn_prefill(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ kc, const bf16_t* __restrict__ vc,
    const int32_t* __restrict__ pos, bf16_t* __restrict__ out, int T, int H, int max_ctx,
    int window, int is_long, float scale, float shift) {
  constexpr int BQ = 128, BK = 64;
  constexpr int KP = DH + 8;   // K and V tile row pitch (bf16)
  constexpr int NKS = DH / 32; // k-steps of the QK product
  constexpr int NDB = DH / 16; // 16-dim blocks of the output
  constexpr int CPT = BK * DH / 8 / 512;   // 16-byte chunks per thread per tile
  __shared__ __attribute__((aligned(16))) bf16_t Ks[BK * KP];
  __shared__ __attribute__((aligned(16))) bf16_t Vs[BK * KP];

  // XCD-aware order: work-group L runs on XCD L % 8, so work item
  // (L % 8) * N/8 + L / 8 puts consecutive items -- the query blocks of one
  // (row, head), which read the same keys and values -- on one XCD and its L2
  int qb, h, b;
  {
    const int nx = gridDim.x, ny = gridDim.y, N = nx * ny * gridDim.z;
    const int L = blockIdx.x + nx * (blockIdx.y + ny * blockIdx.z);
    const int w = (N % 8 == 0) ? (L % 8) * (N / 8) + L / 8 : L;
    qb = w % nx;
    h = (w / nx) % ny;
    b = w / (nx * ny);
  }
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int r16 = lane & 15, g4 = lane >> 4;
  const int d = H * DH;
  const int p0 = pos[b];
  const int qs = qb * BQ;
  const int tq = qs + wv * 16 + r16;   // this lane's query (B-operand column)
  const bool qok = tq < T;
  const int qp = p0 + tq;              // its position
  // this wave's 16 queries: positions wq0 .. wq0 + 15 (all valid iff wall)
  const int wq0 = p0 + qs + wv * 16;
  const bool wall = qs + wv * 16 + 15 < T;
  const int wqn = min(T - (qs + wv * 16), 16);   // valid queries of the wave (may be <= 0)

  bf16x8_t qf[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    uint4 v = qok ? *(const uint4*)(q + (size_t)(b * T + tq) * d + h * DH + ks * 32 + g4 * 8)
                  : make_uint4(0, 0, 0, 0);
    qf[ks] = *(bf16x8_t*)&v;
  }
  const int qpos_lo = p0 + qs;
  const int qpos_hi = p0 + min(qs + BQ, T) - 1;
  const int klo = is_long ? 0 : max(0, qpos_lo - window + 1);
  const int kbeg = klo & ~(BK - 1);
  const int kend = qpos_hi + 1;
  const size_t head = ((size_t)b * H + h) * max_ctx;
  const bf16_t* kh = kc + head * DH;
  const bf16_t* vh = vc + head * DH;
  const float sl2 = scale * 1.4426950408889634f, sh2 = shift * 1.4426950408889634f;
  // ds_read_b64_tr_b16 source row / column of this lane inside a 32-key step
  const int trow = 4 * g4 + (r16 >> 2), tcol = 4 * (r16 & 3);

  floatx4_t o[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) o[i] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
  float lsum = 0.f;

  uint4 kr[CPT], vr[CPT];
  auto fetch = [&](int kb) {
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int c = tid + u * 512;
      const int key = c / (DH / 8), dc = (c % (DH / 8)) * 8;
      const int j = kb + key;
      kr[u] = j < kend ? *(const uint4*)(kh + (size_t)j * DH + dc) : make_uint4(0, 0, 0, 0);
      vr[u] = j < kend ? *(const uint4*)(vh + (size_t)j * DH + dc) : make_uint4(0, 0, 0, 0);
    }
  };
  fetch(kbeg);
  for (int kb = kbeg; kb < kend; kb += BK) {
    __syncthreads();
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int c = tid + u * 512;
      const int key = c / (DH / 8), dc = (c % (DH / 8)) * 8;
      *(uint4*)&Ks[key * KP + dc] = kr[u];
      *(uint4*)&Vs[key * KP + dc] = vr[u];
    }
    __syncthreads();
    if (kb + BK < kend) fetch(kb + BK);   // next tile in flight during the math

    // wave-uniform: any (query, key) of this tile inside the wave's window?
    const bool live = wqn > 0 && kb <= wq0 + wqn - 1 && (is_long || wq0 - (kb + BK - 1) < window);
    if (!live) continue;
    const bool full = wall && kb + BK - 1 <= wq0 && (is_long || wq0 + 15 - kb < window);

    floatx4_t sacc[4];
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      sacc[blk] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const bf16x8_t kf = *(const bf16x8_t*)&Ks[(blk * 16 + r16) * KP + ks * 32 + g4 * 8];
        sacc[blk] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[ks], sacc[blk], 0, 0, 0);
      }
    }
    float pv[4][4];
    if (full) {
#pragma unroll
      for (int blk = 0; blk < 4; ++blk)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pj = __builtin_amdgcn_exp2f(sacc[blk][r] * sl2 - sh2);
          pv[blk][r] = pj;
          lsum += pj;
        }
    } else {
#pragma unroll
      for (int blk = 0; blk < 4; ++blk)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = kb + blk * 16 + g4 * 4 + r;
          const bool ok = qok && j <= qp && (is_long || qp - j < window);
          const float pj = ok ? __builtin_amdgcn_exp2f(sacc[blk][r] * sl2 - sh2) : 0.f;
          pv[blk][r] = pj;
          lsum += pj;
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      uint32_t hi[4], lo[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x0 = pv[2 * i + (e >> 1)][(e & 1) * 2];
        const float x1 = pv[2 * i + (e >> 1)][(e & 1) * 2 + 1];
        hi[e] = pack2(x0, x1);
        lo[e] = pack2(x0 - __uint_as_float(hi[e] << 16), x1 - __uint_as_float(hi[e] & 0xffff0000u));
      }
      const bf16x8_t ph = *(const bf16x8_t*)hi;
      const bf16x8_t pl = *(const bf16x8_t*)lo;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const bf16_t* src = &Vs[(32 * i + trow) * KP + db * 16 + tcol];
        const ap_v4i16 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((ap_lds_v4i16*)src);
        const ap_v4i16 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((ap_lds_v4i16*)(src + 16 * KP));
        const short a8[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
        const bf16x8_t vf = *(const bf16x8_t*)a8;
        o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, ph, o[db], 0, 0, 0);
        o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pl, o[db], 0, 0, 0);
      }
    }
  }
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);
  if (qok) {
    const float inv = 1.f / lsum;
    bf16_t* orow = out + (size_t)(b * T + tq) * d + h * DH;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      uint2 w;
      w.x = pack2(o[db][0] * inv, o[db][1] * inv);
      w.y = pack2(o[db][2] * inv, o[db][3] * inv);
      *(uint2*)(orow + db * 16 + g4 * 4) = w;
    }
  }
}

hipError_t attn_prefill(const bf16_t* q, const bf16_t* kc, const bf16_t* vc, const int32_t* pos,
                        bf16_t* out, int B, int T, int H, int Dh, int max_ctx, int window,
                        bool long_layer, float scale, hipStream_t st) {
  if (B <= 0 || T <= 0) return hipErrorInvalidValue;
  const float shift = scale * (float)Dh * 1.02f;
  dim3 grid((T + 127) / 128, H, B);
  switch (Dh) {
    case 64:
      hipLaunchKernelGGL(k_attn_prefill<64>, grid, dim3(512), 0, st, q, kc, vc, pos, out, T, H,
                         max_ctx, window, (int)long_layer, scale, shift);
      break;
    case 128:
      hipLaunchKernelGGL(k_attn_prefill<128>, grid, dim3(512), 0, st, q, kc, vc, pos, out, T, H,
                         max_ctx, window, (int)long_layer, scale, shift);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace ann
