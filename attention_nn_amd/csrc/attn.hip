// Prefill attention of B x T query rows against the bf16 KV cache
// (model.py:248-254): keep key j for query position p iff j <= p and, on the
// windowed layers, p - j < window.  Scores 0.1 * q.k in fp32, softmax
// weights in fp32 rounded to bf16 for P.V, accumulated in fp32, output rounded
// once to bf16.
#include <math.h>
#include <type_traits>
#include "common.h"
#include "launch.h"

namespace ann {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

// ---- prefill: MFMA flash attention ------------------------------------------
//
// Grid (ceil(T/128), H, B), 512 threads: 8 waves x 16 queries.  K and V tiles
// of BK keys stream through a ring of NS LDS stages: each tile is loaded
// straight into LDS (global_load_lds_dwordx4, 1 KB per wave instruction, no
// register staging) NS - 1 tiles ahead of its use; one barrier per tile.  LDS
// rows are the unpadded DH-element rows of the cache with 16-byte chunk c of
// row r stored at chunk c ^ swz(r), conflict-free on the 64 banks for both
// fragment reads below.  Each wave computes S^T = K Q^T with
// v_mfma_f32_16x16x32_bf16 (keys as rows, its 16 queries as columns) so the
// score fragments are already in the B-operand layout of O^T = V^T P^T: k index
// g*8 + e of a lane maps to key 32i + 4g + e (e < 4) and 32i + 16 + 4g + e - 4
// (e >= 4).  The V^T A-operand comes straight from the row-major V tile through
// ds_read_b64_tr_b16: within each 16-lane group g, output lane m, element e is
// element (m & 3) of the 4-element row addressed by lane 4e + (m >> 2); lane i
// therefore points at key 32i + 4g + (i >> 2) (+16 for the second half), dims
// 16 db + 4 (i & 3), and lane m receives V[32i + 4g + e][16 db + m] for
// e = 0..3.  P enters the MFMA rounded to bf16 (one MFMA per 32-key step), as
// MLX's decomposed attention forms it (softmax output in bf16, then a bf16
// matmul); a bf16 hi + lo pair (two MFMAs, P.V at ~2^-17 relative accuracy)
// measured 7.12 against 7.05 ms for the 64 x 512-token prefill and 29.6
// against 28.6 ms at 16 x 7680.  Softmax: fixed shift, as in the decode kernel
// (|score| <= scale * Dh).  Key tiles entirely outside the causal window of the
// query block are never visited; a wave skips the tiles outside its own 16
// queries' window and evaluates the mask only on tiles that cross the diagonal
// or the window edge.  Keys past the block's last query are loaded as copies of
// that query's own key and value row (finite), and masked.

typedef short ap_v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void ap_lds_void;

// 16-byte chunk swizzle of LDS row r: conflict-free for 16 rows x one chunk
// (the K fragment reads) and for 8 rows x two chunks (the transposed V reads)
template <int DH>
__device__ __forceinline__ int ap_swz(int r) {
  return DH == 128 ? (((r & 7) << 1) | ((r >> 3) & 1)) : ((r >> 1) & 7);
}

template <int N>
__device__ __forceinline__ void ap_wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"i"(N) : "memory");
}

// LDS fragment reads as inline assembly: the compiler's wait insertion treats
// every LDS read as possibly aliasing the loads into LDS still in flight and
// would wait for all of them (the whole ring) before each read; the ring's own
// wait and barrier already order these reads.  Each result is consumed only
// after ap_wait_lgkm on it (LDS reads complete in order).
typedef __attribute__((address_space(3))) const unsigned char ap_lds_cchar;
template <int OFF>
__device__ __forceinline__ bf16x8_t ap_rd_b128(ap_lds_cchar* p) {
  bf16x8_t v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(p), "i"(OFF));
  return v;
}
template <int OFF>
__device__ __forceinline__ ap_v4i16 ap_rd_tr(ap_lds_cchar* p) {
  ap_v4i16 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(p), "i"(OFF));
  return v;
}
// wait until at most N LDS reads are in flight; x (the oldest wanted result)
// is an operand so that its uses stay after the wait
template <int N, typename X>
__device__ __forceinline__ void ap_wait_lgkm(X& x) {
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(x) : "i"(N));
}
template <int I, int N, typename F>
__device__ __forceinline__ void ap_static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    ap_static_for<I + 1, N>(f);
  }
}

template <int DH, int BK, int NS>
constexpr size_t ap_lds_bytes() { return (size_t)NS * 2 * BK * DH * 2; }

// two work-groups per CU (four waves per SIMD, 128 VGPRs) where their rings
// fit the 160 KB of LDS together, else one (256 VGPRs)
template <int DH, int BK, int NS>
constexpr int ap_waves_per_eu() { return ap_lds_bytes<DH, BK, NS>() <= 80 * 1024 ? 4 : 2; }

template <int DH, int BK, int NS>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(ap_waves_per_eu<DH, BK, NS>()))) void k_attn_prefill(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ kc, const bf16_t* __restrict__ vc,
    const int32_t* __restrict__ pos, bf16_t* __restrict__ out, int T, int H, int max_ctx,
    int window, int is_long, float scale, float shift, int lpt) {
  constexpr int BQ = 128;
  constexpr int RB = DH * 2;          // LDS row bytes
  constexpr int TB = BK * RB;         // bytes of one K (or V) tile
  constexpr int LPW = TB / 1024 / 8;  // 1 KB load instructions per wave per K (or V) tile
  static_assert(LPW >= 1 && LPW * 8 * 1024 == TB, "tile split over the waves");
  static_assert(NS >= 2 && NS <= 6, "ring depth");
  constexpr int NKS = DH / 32;        // k-steps of the QK product
  constexpr int NDB = DH / 16;        // 16-dim blocks of the output
  constexpr int NBLK = BK / 16;       // 16-key blocks of a tile
  constexpr int NI = BK / 32;         // 32-key steps of the PV product
  extern __shared__ __attribute__((aligned(16))) unsigned char ap_smem[];

  // Work order.  Work-group L runs on XCD L % 8.
  //  * lpt (host: the NP (row, head) pairs of one query block fit the
  //    resident work-groups): the query blocks of a sequence differ up to
  //    nx-fold in key tiles, so the longest go first (work-group L takes
  //    query block nx - 1 - L / NP of pair L % NP) and the short ones fill
  //    the slots the long ones leave; with NP a multiple of 8 every block of
  //    a pair lands on one XCD.  64 x 512 tokens: 81 -> 65 us per layer
  //    (dispatched by pair it took 78 us for ~41 us of work per slot);
  //    16 x 7680: 656 -> 620 us.
  //  * otherwise (cfg5: 1536 pairs, three rounds per block): work item
  //    (L % 8) * N/8 + L / 8 -- consecutive items, the query blocks of one
  //    pair, run together on one XCD and share its L2 (longest-first measured
  //    672 -> 707 us there: a pair's blocks rounds apart re-read its keys).
  int qb, h, b;
  {
    const int nx = gridDim.x, ny = gridDim.y, NP = ny * gridDim.z, N = nx * NP;
    const int L = blockIdx.x + nx * (blockIdx.y + ny * blockIdx.z);
    if (lpt) {
      qb = nx - 1 - L / NP;
      h = (L % NP) % ny;
      b = (L % NP) / ny;
    } else {
      const int w = (N % 8 == 0) ? (L % 8) * (N / 8) + L / 8 : L;
      qb = w % nx;
      h = (w / nx) % ny;
      b = w / (nx * ny);
    }
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

  // q fragments: unconditional loads issued ahead of the ring's (a query past
  // T reads row T - 1: its scores are always masked and its output not stored)
  bf16x8_t qf[NKS];
  const bf16_t* qrow = q + (size_t)(b * T + min(tq, T - 1)) * d + h * DH + g4 * 8;
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) qf[ks] = *(const bf16x8_t*)(qrow + ks * 32);
  __builtin_amdgcn_sched_barrier(0);
  const int qpos_lo = p0 + qs;
  const int qpos_hi = p0 + min(qs + BQ, T) - 1;
  const int klo = is_long ? 0 : max(0, qpos_lo - window + 1);
  const int kbeg = klo & ~(BK - 1);
  const int kend = qpos_hi + 1;
  const int ntile = (kend - kbeg + BK - 1) / BK;
  const size_t head = ((size_t)b * H + h) * max_ctx;
  const bf16_t* kh = kc + head * DH;
  const bf16_t* vh = vc + head * DH;
  const float sl2 = scale * 1.4426950408889634f, sh2 = shift * 1.4426950408889634f;

  // the rows and logical chunks this lane loads: byte o of a tile is row
  // o / RB, stored chunk (o % RB) / 16, logical chunk stored ^ swz(row)
  int lrow[LPW], lcol[LPW];
#pragma unroll
  for (int u = 0; u < LPW; ++u) {
    const int o = (wv * LPW + u) * 1024 + lane * 16;
    lrow[u] = o / RB;
    lcol[u] = (((o % RB) >> 4) ^ ap_swz<DH>(o / RB)) * 8;
  }
  auto issue = [&](int t) {
    const int kb = kbeg + t * BK;
    unsigned char* st = ap_smem + (size_t)(t % NS) * 2 * TB;
#pragma unroll
    for (int u = 0; u < LPW; ++u) {
      const size_t j = (size_t)min(kb + lrow[u], kend - 1) * DH + lcol[u];
      __builtin_amdgcn_global_load_lds(kh + j, (ap_lds_void*)(st + (wv * LPW + u) * 1024), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(vh + j, (ap_lds_void*)(st + TB + (wv * LPW + u) * 1024), 16,
                                       0, 0);
    }
  };
  // wait until at most n tiles of this wave's loads are still in flight
  auto wait_tiles = [&](int n) {
    if constexpr (NS > 5) { if (n >= 4) { ap_wait_vm<8 * LPW>(); return; } }
    if constexpr (NS > 4) { if (n >= 3) { ap_wait_vm<6 * LPW>(); return; } }
    if constexpr (NS > 3) { if (n >= 2) { ap_wait_vm<4 * LPW>(); return; } }
    if constexpr (NS > 2) { if (n >= 1) { ap_wait_vm<2 * LPW>(); return; } }
    ap_wait_vm<0>();
  };

  // per-lane parts of the fragment addresses (the swizzle of rows r16 / trow)
  const int kx = ap_swz<DH>(r16);
  const int trow = 4 * g4 + (r16 >> 2), tcol = 4 * (r16 & 3);
  const int vx = ap_swz<DH>(trow);

  floatx4_t o[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) o[i] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
  float lsum = 0.f;

  // prologue: NS - 1 tiles, unconditionally (a tile past the last reads the
  // clamped row), so that the waits below have fixed counts
#pragma unroll
  for (int t = 0; t < NS - 1; ++t) issue(t);
  for (int t = 0; t < ntile; ++t) {
    const int kb = kbeg + t * BK;
    wait_tiles(min(NS - 2, ntile - 1 - t));   // this wave's part of tile t is in LDS
    __syncthreads();                            // every wave's; stage (t - 1) % NS is free
    if (t + NS - 1 < ntile) issue(t + NS - 1);

    // wave-uniform: any (query, key) of this tile inside the wave's window?
    const bool live = wqn > 0 && kb <= wq0 + wqn - 1 && (is_long || wq0 - (kb + BK - 1) < window);
    if (!live) continue;
    const bool full = wall && kb + BK - 1 <= wq0 && (is_long || wq0 + 15 - kb < window);
    const unsigned char* ks_ = ap_smem + (size_t)(t % NS) * 2 * TB;
    const unsigned char* vs_ = ks_ + TB;

    ap_lds_cchar* kst = (ap_lds_cchar*)ks_ + r16 * RB;
    floatx4_t sacc[NBLK];
#pragma unroll
    for (int blk = 0; blk < NBLK; ++blk) sacc[blk] = (floatx4_t){0.f, 0.f, 0.f, 0.f};
    // K fragments: one k-step (NBLK reads) ahead of its MFMAs
    bf16x8_t kf[2][NBLK];
    ap_static_for<0, NBLK>([&](auto bc) __attribute__((always_inline)) {
      constexpr int blk = decltype(bc)::value;
      kf[0][blk] = ap_rd_b128<blk * 16 * RB>(kst + ((g4 ^ kx) << 4));
    });
    ap_static_for<0, NKS>([&](auto kc_) __attribute__((always_inline)) {
      constexpr int ks = decltype(kc_)::value;
      if constexpr (ks + 1 < NKS) {
        ap_static_for<0, NBLK>([&](auto bc) __attribute__((always_inline)) {
          constexpr int blk = decltype(bc)::value;
          kf[(ks + 1) & 1][blk] =
              ap_rd_b128<blk * 16 * RB>(kst + ((((ks + 1) * 4 + g4) ^ kx) << 4));
        });
      }
      constexpr int ahead = ks + 1 < NKS ? NBLK : 0;   // reads issued after this k-step's
      ap_static_for<0, NBLK>([&](auto bc) __attribute__((always_inline)) {
        constexpr int blk = decltype(bc)::value;
        ap_wait_lgkm<ahead + NBLK - 1 - blk>(kf[ks & 1][blk]);
        sacc[blk] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks & 1][blk], qf[ks], sacc[blk], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);   // keep each wait next to its MFMA
      });
    });
    float pv[NBLK][4];
    if (full) {
#pragma unroll
      for (int blk = 0; blk < NBLK; ++blk)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pj = __builtin_amdgcn_exp2f(sacc[blk][r] * sl2 - sh2);
          pv[blk][r] = pj;
          lsum += pj;
        }
    } else {
#pragma unroll
      for (int blk = 0; blk < NBLK; ++blk)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = kb + blk * 16 + g4 * 4 + r;
          const bool ok = qok && j <= qp && (is_long || qp - j < window);
          const float pj = ok ? __builtin_amdgcn_exp2f(sacc[blk][r] * sl2 - sh2) : 0.f;
          pv[blk][r] = pj;
          lsum += pj;
        }
    }
    ap_lds_cchar* vst = (ap_lds_cchar*)vs_ + trow * RB + (tcol & 7) * 2;
    ap_static_for<0, NI>([&](auto ic) __attribute__((always_inline)) {
      constexpr int i = decltype(ic)::value;
      // every V fragment of this 32-key step in flight before the P packing
      ap_v4i16 v0[NDB], v1[NDB];
      ap_static_for<0, NDB>([&](auto dc) __attribute__((always_inline)) {
        constexpr int db = decltype(dc)::value;
        ap_lds_cchar* src = vst + (((2 * db + (tcol >> 3)) ^ vx) << 4);
        v0[db] = ap_rd_tr<32 * i * RB>(src);
        v1[db] = ap_rd_tr<(32 * i + 16) * RB>(src);
      });
      uint32_t pw[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        pw[e] = pack2(pv[2 * i + (e >> 1)][(e & 1) * 2], pv[2 * i + (e >> 1)][(e & 1) * 2 + 1]);
      const bf16x8_t ph = *(const bf16x8_t*)pw;
      ap_static_for<0, NDB>([&](auto dc) __attribute__((always_inline)) {
        constexpr int db = decltype(dc)::value;
        ap_wait_lgkm<2 * (NDB - 1 - db)>(v0[db]);
        ap_wait_lgkm<2 * (NDB - 1 - db)>(v1[db]);
        const short a8[8] = {v0[db][0], v0[db][1], v0[db][2], v0[db][3],
                             v1[db][0], v1[db][1], v1[db][2], v1[db][3]};
        const bf16x8_t vf = *(const bf16x8_t*)a8;
        o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, ph, o[db], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      });
    });
  }
  ap_wait_vm<0>();   // no load into LDS outlives the work-group
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

template <int DH, int BK, int NS>
static hipError_t attn_prefill_launch(dim3 grid, hipStream_t st, const bf16_t* q, const bf16_t* kc,
                                      const bf16_t* vc, const int32_t* pos, bf16_t* out, int T,
                                      int H, int max_ctx, int window, bool long_layer, float scale,
                                      float shift) {
  constexpr size_t lds = ap_lds_bytes<DH, BK, NS>();
  static hipError_t attr = hipFuncSetAttribute((const void*)k_attn_prefill<DH, BK, NS>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (attr != hipSuccess) return attr;
  // longest query blocks first when one block's (row, head) pairs fit the
  // resident work-groups (ap_waves_per_eu: 4 waves per SIMD = two 8-wave
  // work-groups per CU, else one)
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
  }
  const long long resident = (long long)cus * (ap_waves_per_eu<DH, BK, NS>() / 2);
  const int lpt = (long long)grid.y * grid.z <= resident ? 1 : 0;
  hipLaunchKernelGGL((k_attn_prefill<DH, BK, NS>), grid, dim3(512), lds, st, q, kc, vc, pos, out, T,
                     H, max_ctx, window, (int)long_layer, scale, shift, lpt);
  return hipGetLastError();
}

hipError_t attn_prefill(const bf16_t* q, const bf16_t* kc, const bf16_t* vc, const int32_t* pos,
                        bf16_t* out, int B, int T, int H, int Dh, int max_ctx, int window,
                        bool long_layer, float scale, hipStream_t st) {
  if (B <= 0 || T <= 0) return hipErrorInvalidValue;
  const float shift = scale * (float)Dh * 1.02f;
  dim3 grid((T + 127) / 128, H, B);
  // ring of two 32-key stages: deeper rings (3 to 5 stages, or 64-key tiles
  // with one work-group per CU) measured equal or slower
#define AP_ARGS grid, st, q, kc, vc, pos, out, T, H, max_ctx, window, long_layer, scale, shift
  switch (Dh) {
    case 64:
      return attn_prefill_launch<64, 64, 2>(AP_ARGS);
    case 128:
      return attn_prefill_launch<128, 32, 2>(AP_ARGS);
    default:
      return hipErrorInvalidValue;
  }
#undef AP_ARGS
}

}  // namespace ann
