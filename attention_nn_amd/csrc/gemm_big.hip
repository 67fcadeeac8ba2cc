// Large projections y = a @ W^T (W stored (N, K) bf16) of the prefill and the
// training forward: 256 x 256 (or 256 x 192) output tiles of four waves of
// 128 x 128 (128 x 96), one work-group (one wave per SIMD) per CU,
// v_mfma_f32_16x16x32_bf16.  The projection routing sends the fc (relu^2),
// o-proj (attention residual) and proj (MLP residual) projections here (see
// gemm_big_routes for the measurements); it serves the plain and QKV
// epilogues as well when called directly.
//
// Main loop (K tiles of 64, two LDS stages, one barrier per K tile):
//   * the 256 accumulators of a wave live in AGPRs: the MFMA is issued as
//     inline assembly whose accumulator operand is an AGPR ("+a").  With the
//     compiler builtin the accumulators move between AGPRs and VGPRs inside the
//     loop (368 v_accvgpr moves per K tile, measured ~10% slower);
//   * the fragments are read with volatile inline ds_read_b128 in a fixed
//     order -- the first k-step's eight W fragments and the first A fragment,
//     then the second k-step's W fragments -- and each A fragment one group of
//     eight MFMAs ahead of its use, with hand-placed s_waitcnt (the compiler's
//     scheduler otherwise reads every A fragment right before its MFMAs and
//     waits for it);
//   * each of the 16 MFMA groups of a K tile first stores one 16-byte chunk per
//     thread of the next K tile into the other LDS stage and refills that
//     register with the tile after it, so the tile traffic hides behind the
//     MFMAs.  All of these are unconditional (past the last K tile they re-read
//     it and fill the stage no later iteration reads): a branch there makes the
//     compiler wait on every load in flight.  The prologue issues the second
//     tile's loads in the loop's order, so the loop's waits stay vmcnt(15).
//   * LDS tiles are unpadded 128-byte rows with chunk c of row r at slot
//     c ^ ((r >> 1) & 7): conflict-free for the chunk stores and the
//     16-row fragment reads.
// The MFMA operands are swapped (C^T = W A^T) so that a lane holds four
// consecutive columns of one row.  Epilogue: the tile is rounded to bf16 (every
// epilogue here starts from bf16(y), as the reference's eager ops do; relu^2
// is applied at this point) into LDS (row pitch 264: the 8-byte writes of 16
// rows spread over the banks), then each thread handles 16-byte row chunks:
// plain / relu^2 copies, the residual mixes (x, x0 read and x written as
// 16-byte words, the first batch loaded before the staging), or the QKV
// epilogue of each 128-column half (QK-norm, RoPE, q and KV-cache writes).
// With one wave per SIMD nothing hides the epilogue's VALU work, so every
// eager rounding is a packed pair conversion (v_cvt_pk_bf16_f32): per-work-
// group stamps of the 64 x 512-token prefill put the fc epilogue at 5.7-7.5
// us per tile after this, 7.3 before (main loop ~21 us).  Work-group i
// runs on XCD i % 8; each XCD takes a contiguous range of tiles, N-fastest, so
// the N tiles of an M block share its A rows in that XCD's L2.
// Measured against the four prefill shapes (M = 32768) with a plain store:
// 0.81 / 0.70 / 0.96 / 1.04 PFLOP/s for N x K = 2304 x 768, 768 x 768,
// 3072 x 768, 768 x 3072 (hipBLASLt: 0.87 / 0.83 / 1.17 / 1.29).
#include <stdlib.h>
#include <type_traits>
#include "common.h"
#include "epilogue.h"
#include "launch.h"

namespace ann {

namespace {

constexpr int BG_BM = 256, BG_BN = 256, BG_BK = 64;   // BG_BN: the widest tile
constexpr int BG_EP = 264;   // bf16 row pitch of the staged output tile
#ifndef BG_EB
#define BG_EB 8              // residual epilogue: 16-byte chunks per thread loaded at once
#endif
constexpr size_t BG_LDS_MAIN = (size_t)2 * (BG_BM + BG_BN) * BG_BK * 2;
constexpr size_t BG_LDS_EPI = (size_t)BG_BM * BG_EP * 2;
constexpr size_t BG_LDS = BG_LDS_MAIN > BG_LDS_EPI ? BG_LDS_MAIN : BG_LDS_EPI;

typedef __bf16 bg_bf16x8 __attribute__((ext_vector_type(8)));
typedef float bg_floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned bg_u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) char bg_lds_char;

template <int I, int N, typename F>
__device__ __forceinline__ void bg_static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    bg_static_for<I + 1, N>(f);
  }
}

__device__ __forceinline__ int bg_off(int r, int c) { return r * BG_BK + ((c ^ ((r >> 1) & 7)) << 3); }

__device__ __forceinline__ void bg_mfma(bg_floatx4& acc, const bg_bf16x8& a, const bg_bf16x8& b) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

template <int OFF>
__device__ __forceinline__ bg_bf16x8 bg_lds_read(const bg_lds_char* p) {
  bg_bf16x8 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(p), "i"(OFF));
  return v;
}

template <int N>
__device__ __forceinline__ void bg_wait_lgkm() {
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(N) : "memory");
}

}  // namespace


template <int EPI, int BN>
__global__ __launch_bounds__(256, 1) void k_gemm_big(const bf16_t* A, int lda, const bf16_t* W,
                                                     int M, int N, int K, EpiArgs ea) {
  static_assert(BN == 256 || BN == 192, "tile width");
  static_assert(EPI != EPI_QKV || BN == 256, "the QKV epilogue takes 128-column head halves");
  constexpr int NJ = BN / 32;    // 16-column blocks of a wave (two waves across the tile)
  constexpr int NWU = BN / 32;   // W chunks per thread and K tile
  constexpr int CPR = BN / 8;    // 16-byte chunks per output row
  extern __shared__ __attribute__((aligned(16))) bf16_t smem[];
  auto As = [&](int s) { return smem + s * BG_BM * BG_BK; };
  auto Ws = [&](int s) { return smem + 2 * BG_BM * BG_BK + s * BN * BG_BK; };
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv >> 1, wn = wv & 1;
  const int ntm = (M + BG_BM - 1) / BG_BM, ntn = N / BN, nt = ntm * ntn;
  const int per = (nt + 7) / 8;
  const int t = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (t >= nt) return;
  const int tm = t / ntn, tn = t % ntn;
  const int m0 = tm * BG_BM, n0 = tn * BN;
  const int KT = K / BG_BK;

  // staged K-tile chunks: chunk g of a thread is operand g & 1 (A, W), row
  // block g >> 1 (rows (tid >> 3) + 32 u), 16-byte column tid & 7
  bg_u32x4 ra[8], rw[8];
  const int crow = tid >> 3, cc = tid & 7;
  auto gload1 = [&](int op, int u, int kt) {
    const int row = crow + 32 * u;
    if (op == 0)
      ra[u] = *(const bg_u32x4*)(A + (size_t)min(m0 + row, M - 1) * lda + kt * BG_BK + cc * 8);
    else if (u < NWU)
      rw[u] = *(const bg_u32x4*)(W + (size_t)(n0 + row) * K + kt * BG_BK + cc * 8);
  };
  auto lstore1 = [&](int op, int u, int s) {
    const int row = crow + 32 * u;
    if (op == 0) *(bg_u32x4*)(As(s) + bg_off(row, cc)) = ra[u];
    else if (u < NWU) *(bg_u32x4*)(Ws(s) + bg_off(row, cc)) = rw[u];
  };

  bg_floatx4 acc[8][NJ];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = (bg_floatx4){0.f, 0.f, 0.f, 0.f};
  const int r16 = lane & 15, kg = lane >> 4;

  // prologue: tile 0 into stage 0, tile 1 (clamped) in flight in the
  // loop's order, each load pinned in place
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    gload1(0, u, 0);
    gload1(1, u, 0);
  }
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    lstore1(0, u, 0);
    lstore1(1, u, 0);
  }
  bg_static_for<0, 16>([&](auto gc) __attribute__((always_inline)) {
    constexpr int g = decltype(gc)::value;
    gload1(g & 1, g >> 1, min(1, KT - 1));
    asm volatile("" ::: "memory");
  });
  __syncthreads();

  for (int kt = 0; kt < KT; ++kt) {
    const int s = kt & 1;
    const bf16_t* as = As(s) + (wm * 128 + r16) * BG_BK;
    const bf16_t* ws = Ws(s) + (wn * (BN / 2) + r16) * BG_BK;
    const int ch0 = kg ^ ((r16 >> 1) & 7), ch1 = (4 + kg) ^ ((r16 >> 1) & 7);
    const bg_lds_char* pa0 = (const bg_lds_char*)(as + (ch0 << 3));
    const bg_lds_char* pa1 = (const bg_lds_char*)(as + (ch1 << 3));
    const bg_lds_char* pb0 = (const bg_lds_char*)(ws + (ch0 << 3));
    const bg_lds_char* pb1 = (const bg_lds_char*)(ws + (ch1 << 3));
    bg_bf16x8 b0[NJ], b1[NJ];
    bg_static_for<0, NJ>([&](auto jc) __attribute__((always_inline)) {
      constexpr int j = decltype(jc)::value;
      b0[j] = bg_lds_read<j * 16 * BG_BK * 2>(pb0);
    });
    bg_bf16x8 a = bg_lds_read<0>(pa0);
    bg_static_for<0, NJ>([&](auto jc) __attribute__((always_inline)) {
      constexpr int j = decltype(jc)::value;
      b1[j] = bg_lds_read<j * 16 * BG_BK * 2>(pb1);
    });
    // b0 and a; the b1 reads may still fly.  A wave's LDS reads return in
    // issue order, so lgkmcnt(NJ) leaves only the last NJ issued (the b1
    // reads) outstanding; any scalar load the compiler has in flight counts
    // on the same counter and only makes the wait stricter.  The lgkmcnt(0)
    // after each MFMA group covers the next A fragment the same way.
    bg_wait_lgkm<NJ>();
    bg_static_for<0, 16>([&](auto gc) __attribute__((always_inline)) {
      constexpr int g = decltype(gc)::value;
      constexpr int i = g & 7, kh = g >> 3;
      bg_bf16x8 an = a;
      if constexpr (g < 15) {
        constexpr int ni = (g + 1) & 7;
        an = ((g + 1) >> 3) ? bg_lds_read<ni * 16 * BG_BK * 2>(pa1)
                            : bg_lds_read<ni * 16 * BG_BK * 2>(pa0);
      }
      lstore1(g & 1, g >> 1, s ^ 1);
      gload1(g & 1, g >> 1, min(kt + 2, KT - 1));
      asm volatile("" ::: "memory");
#pragma unroll
      for (int j = 0; j < NJ; ++j) bg_mfma(acc[i][j], kh ? b1[j] : b0[j], a);
      if constexpr (g < 15) bg_wait_lgkm<0>();
      a = an;
    });
    // After the loop the accumulators leave their AGPRs through
    // v_accvgpr_read / _mov (the epilogue and the register allocator's
    // copies).  The compiler's hazard recognizer does not see these MFMAs
    // (inline assembly), so the wait states an XDL result needs before a VALU
    // or v_accvgpr instruction reads it are placed here by hand: the CDNA3 /
    // CDNA4 ISA's MAI dependency table asks NumPasses + 3 (+1 on gfx950) for
    // "XDL write VGPR -> VALU read", 12 for the 8-pass
    // v_mfma_f32_16x16x32_bf16; three s_nop 7 give 24.  In the loop body,
    // after the last MFMA group, every copy on the loop's exit path comes
    // after them; they issue while the MFMA pipe drains the group, before
    // the barrier.
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
    __syncthreads();
  }

  // residual epilogues: x (and x0) chunks of the first batch loaded before the
  // staging (chunk q = tid + 256 u is row q / CPR, columns 8 (q % CPR); rows
  // past M read row M - 1 and are never stored)
  constexpr bool RES = EPI == EPI_RESID_ATTN || EPI == EPI_RESID_MLP;
  static_assert(!RES || CPR % BG_EB == 0, "whole batches");
  bg_u32x4 xv[2][BG_EB], zv[2][BG_EB];
  auto res_load = [&](int b) {
#pragma unroll
    for (int e = 0; e < BG_EB; ++e) {
      const int q = tid + 256 * (b * BG_EB + e);
      const size_t i = (size_t)min(m0 + q / CPR, M - 1) * ea.ldr + n0 + (q % CPR) * 8;
      xv[b & 1][e] = *(const bg_u32x4*)(ea.x + i);
      if constexpr (EPI == EPI_RESID_ATTN) zv[b & 1][e] = *(const bg_u32x4*)(ea.x0 + i);
    }
  };
  if constexpr (RES) res_load(0);
  QkvRows<BG_BM> pr;
  if constexpr (EPI == EPI_QKV) qkv_prefetch<BG_BM>(ea, m0, M, tid, pr);
  // ---- stage bf16(y): lane holds row m = block row + r16, columns 4 kg ..
  bf16_t* st = smem;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int ml = wm * 128 + i * 16 + r16, nl = wn * (BN / 2) + j * 16 + 4 * kg;
      const bg_floatx4 v = acc[i][j];
      uint2 w;
      if constexpr (EPI == EPI_RELU2)   // relu^2 applied here: the copy below only moves bytes
        w = make_uint2(relu2_pair(v[0], v[1]), relu2_pair(v[2], v[3]));
      else
        w = make_uint2(pack2(v[0], v[1]), pack2(v[2], v[3]));
      *(uint2*)(st + ml * BG_EP + nl) = w;
    }
  __syncthreads();

  if constexpr (EPI == EPI_QKV) {
    qkv_tile_epilogue<BG_BM, BG_EP>(ea, st, m0, n0, M, tid, pr);
    qkv_tile_epilogue<BG_BM, BG_EP>(ea, st + 128, m0, n0 + 128, M, tid, pr);
    return;
  } else {
    // 16-byte row chunks: chunk q = tid + 256 u is row q / CPR, columns 8 (q % CPR)
    if constexpr (RES) {
      // batch b + 1's loads fly while batch b is mixed and stored
      float lam[5];
#pragma unroll
      for (int e = 0; e < 5; ++e) lam[e] = ea.lam[e];
#pragma unroll
      for (int b = 0; b < CPR / BG_EB; ++b) {
        if (b + 1 < CPR / BG_EB) res_load(b + 1);
#pragma unroll
        for (int e = 0; e < BG_EB; ++e) {
          const int q = tid + 256 * (b * BG_EB + e);
          const int ml = q / CPR, c8 = (q % CPR) * 8;
          const bg_u32x4 y = *(const bg_u32x4*)(st + ml * BG_EP + c8);
          const bg_u32x4 x = xv[b & 1][e];
          bg_u32x4 o;
#pragma unroll
          for (int f = 0; f < 4; ++f) {
            if constexpr (EPI == EPI_RESID_ATTN) o[f] = mix_attn_pair(lam, x[f], zv[b & 1][e][f], y[f]);
            else o[f] = mix_mlp_pair(lam, x[f], y[f]);
          }
          if (m0 + ml < M) *(bg_u32x4*)(ea.x + (size_t)(m0 + ml) * ea.ldr + n0 + c8) = o;
        }
      }
      return;
    }
    // plain / relu^2 (already applied): 16-byte row chunks, eight LDS reads
    // in flight per thread; the fc output goes out with non-temporal stores
    // (it is read back only by the next projection; 10 us less per fc call)
    static_assert(CPR % 8 == 0, "whole batches");
#pragma unroll
    for (int u0 = 0; u0 < CPR; u0 += 8) {
      bg_u32x4 w[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int q = tid + 256 * (u0 + e);
        w[e] = *(const bg_u32x4*)(st + (q / CPR) * BG_EP + (q % CPR) * 8);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int q = tid + 256 * (u0 + e);
        const int m = m0 + q / CPR, n = n0 + (q % CPR) * 8;
        if (m < M) {
          bg_u32x4* dst = (bg_u32x4*)(ea.out + (size_t)m * ea.ldo + n);
          if constexpr (EPI == EPI_RELU2) __builtin_nontemporal_store(w[e], dst);
          else *dst = w[e];
        }
      }
    }
  }
}

static int big_cus() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
  }
  return cus;
}

// Whether the projection routing (gemm()) sends (epi, M, N) here.  In the
// 64 x 512-token prefill, per layer against the two-work-groups-per-CU tiles
// of k_gemm_2w (rocprof, one box): fc (relu^2) 185 us here; o-proj (attention
// residual) 79 us here with 192-column tiles (103 with 256, 108 in k_gemm_2w);
// proj (MLP residual) 159 us here with 192-column tiles against 199 in
// k_gemm_2w.  QKV: 165 us here against 150 in k_gemm_2w at 64 x 512 tokens,
// whose 1152 tiles leave the fifth round of 256 CUs half empty; with whole
// rounds it wins (16 x 7680 tokens: 4320 tiles, 565 -> 535 us; d 1536 at
// 128 x 1024: 9216 tiles, 2072 -> 1816 us), so QKV comes here when the last
// round's idle CUs are under 5% of all rounds.  The kernel still serves every
// epilogue of gemm_big() when called directly.
bool gemm_big_routes(int epi, int M, int N) {
  if (epi == EPI_RELU2 || epi == EPI_RESID_ATTN || epi == EPI_RESID_MLP) return true;
  if (epi != EPI_QKV || N % BG_BN) return false;
  const long long cus = big_cus(), tiles = (long long)((M + BG_BM - 1) / BG_BM) * (N / BG_BN);
  const long long slots = (tiles + cus - 1) / cus * cus;
  return (slots - tiles) * 20 < slots;
}

// Tile width for an M x N output: 256 or 192 columns, whichever needs fewer
// CU-rounds times columns (one work-group per CU), a 192-column tile counted
// 15% dearer per column (less reuse of each A tile: the cfg4 fc shape, 480 x 16
// tiles of 192 against 480 x 12 of 256, measured 818 against 713 us).  N = 768
// at M = 32768: 384 tiles of 256 fill 1.5 rounds of 256 CUs, 512 tiles of 192
// two whole rounds (o-proj 79 against 103 us).  The QKV epilogue needs 256
// (head halves).
// ANN_GEMM_BIG_BN=256 / 192 forces one where it divides N (read once per
// process).
static int big_bn(int epi, int M, int N) {
  static int force = -1;
  if (force < 0) {
    const char* e = getenv("ANN_GEMM_BIG_BN");
    force = e ? atoi(e) : 0;
  }
  const int cus = big_cus();
  const bool ok192 = epi != EPI_QKV && N % 192 == 0, ok256 = N % 256 == 0;
  if (!ok192) return 256;
  if (!ok256) return 192;
  if (force == 192 || force == 256) return force;
  const long long ntm = (M + BG_BM - 1) / BG_BM;
  auto rounds = [&](int bn) { return (ntm * (N / bn) + cus - 1) / cus; };
  return rounds(192) * 192 * 115 < rounds(256) * 256 * 100 ? 192 : 256;
}

// Whether gemm_big can take (epi, M, N, K): whole 256- or 192-column tiles,
// 64-deep K tiles, 16-byte aligned rows and outputs, and enough tiles (at
// least 96) for the one-work-group-per-CU kernel to fill the chip.
bool gemm_big_fits(int epi, const bf16_t* A, int lda, int M, int N, int K, const EpiArgs& ea) {
  if (M < 512 || N % 64 || K % BG_BK || K < BG_BK || lda % 8 || ((uintptr_t)A & 15)) return false;
  const int bn = big_bn(epi, M, N);
  if (N % bn) return false;
  if ((long long)((M + BG_BM - 1) / BG_BM) * (N / bn) < 96) return false;
  switch (epi) {
    case EPI_STORE:
    case EPI_RELU2:
      return ea.out && ea.ldo % 8 == 0 && ((uintptr_t)ea.out & 15) == 0;
    case EPI_RESID_ATTN:
      return ea.x && ea.x0 && ea.lam && ea.ldr % 8 == 0 &&
             (((uintptr_t)ea.x | (uintptr_t)ea.x0) & 15) == 0;
    case EPI_RESID_MLP:
      return ea.x && ea.lam && ea.ldr % 8 == 0 && ((uintptr_t)ea.x & 15) == 0;
    case EPI_QKV:
      return true;   // gemm_qkv_fits has been checked by the caller
    default:
      return false;
  }
}

template <int EPI, int BN>
static hipError_t launch_big(const bf16_t* A, int lda, const bf16_t* W, int M, int N, int K,
                             const EpiArgs& ea, hipStream_t st) {
  static bool attr = false;
  if (!attr) {
    const hipError_t e = hipFuncSetAttribute((const void*)k_gemm_big<EPI, BN>,
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             (int)BG_LDS);
    if (e != hipSuccess) return e;
    attr = true;
  }
  const int nt = ((M + BG_BM - 1) / BG_BM) * (N / BN);
  const int grid = (nt + 7) / 8 * 8;
  hipLaunchKernelGGL((k_gemm_big<EPI, BN>), dim3(grid), dim3(256), BG_LDS, st, A, lda, W, M, N, K,
                     ea);
  return hipGetLastError();
}

hipError_t gemm_big(int epi, const bf16_t* A, int lda, const bf16_t* W, int M, int N, int K,
                    const EpiArgs& ea, hipStream_t st) {
  if (!gemm_big_fits(epi, A, lda, M, N, K, ea)) return hipErrorInvalidValue;
  const bool w192 = big_bn(epi, M, N) == 192;
  switch (epi) {
#define ANN_BIG_CASE(E)                                                              \
  case E:                                                                            \
    return w192 ? launch_big<E, 192>(A, lda, W, M, N, K, ea, st)                     \
                : launch_big<E, 256>(A, lda, W, M, N, K, ea, st);
    ANN_BIG_CASE(EPI_STORE)
    ANN_BIG_CASE(EPI_RELU2)
    ANN_BIG_CASE(EPI_RESID_ATTN)
    ANN_BIG_CASE(EPI_RESID_MLP)
#undef ANN_BIG_CASE
    case EPI_QKV: return launch_big<EPI_QKV, 256>(A, lda, W, M, N, K, ea, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ann

