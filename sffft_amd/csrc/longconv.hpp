// Multi-pass causal long convolution for lengths beyond one CU's LDS.
//
//   y[b,h,n] = sum_{m<=n} u[b,h,m] * k[h,n-m],   n < L,   N = 2L = NC * NR,  NR = R0 * R1
//
// The reference stops at L = 8192, whose transform fits one block's shared memory, and
// lists "four-step with one HBM transpose pass" as the way to longer sequences
// (README.md:175). Here the length-N transform is split into a column transform of
// radix NC (16, 32 or 64) and row transforms of length NR (256..4096), with the
// intermediate in HBM:
//
//   position  n = n1*NR + n2,   frequency  k = k1 + NC*k2,   w_N = exp(-2 pi i / N)
//   pass A (columns)  T[k1][n2] = w_N^(n2 k1)/sqrt(NC) * sum_{n1 < NC/2} w_NC^(n1 k1) x[n1*NR + n2]
//   pass B (rows)     per row k1: forward DFT over n2, times the spectrum K[k1 + NC*k2], inverse
//                     DFT over k2, times w_N^(n2 k1)/sqrt(NC), in the conjugated domain:
//                     U[k1][n2] = conj(IDFT(DFT(T[k1]) * K[k1 + NC*.])) * w_N^(n2 k1) / sqrt(NC)
//   pass C (columns)  y[n1*NR + n2] = conj(sum_k1 w_NC^(n1 k1) U[k1][n2]),  n1 < NC/2 only
//
// Two batch rows of one channel travel as the real and imaginary parts of one complex
// sequence x (as in the wave pipeline), so y_a = Re and y_b = Im of the result. Only the
// first NC/2 rows of x are non-zero (the zero padding to 2L), so pass A contracts over
// them alone, and pass C computes only the first L outputs.
//
// Each pass is a chain of v_mfma_f32_16x16x32_f16 contractions with the complex-K
// interleave of fftconv.hpp. Pass B is the wave pipeline's schedule (fftconv_wave.hpp:
// one wavefront per row, every stage in VGPRs, LDS-resident DFT fragments and twiddle
// tables) with a full first stage (the row input is complex and dense), a full last
// stage, the row's slice of the spectrum read from global memory, and the N-level
// twiddle applied to the result before it is stored.
//
// Intermediate: T and U share one workspace, [pair][k1][n2] complex fp16 (4 bytes per
// point, 4N bytes per pair); U overwrites T row by row. The batch runs in chunks of whole
// channels (three launches per chunk) sized by the caller's workspace: a workspace that
// fits the Infinity Cache keeps T and U out of HBM. Every value that enters an MFMA
// is fp16 anyway, so storing fp16 adds no rounding: with fp32 I/O the input enters
// pass A as an fp16 value plus its fp16 remainder, and there are as many fp16
// roundings between input and output as in a three-stage single-pass plan.
//
// Circular convolution of period N (CIRC): y[n] = sum_{m<N} x[m] k[(n - m) mod N], rows of
// length N. The same passes, with pass A contracting over all NC rows and pass C storing
// all of them; the spectrum is the DFT of the unpadded length-N filter.
//
// HBM traffic per pair: pass A reads the two input rows and writes T (4N), pass B reads
// and rewrites it (8N) and its channel's spectrum (8N per channel, shared by the B/2
// pairs through L2), pass C reads U (4N) and writes the two output rows.
#pragma once
#include "fftconv_wave.hpp"

// k0 strips per phase-2 step of the row pass (pass B)
#ifndef LONG_ROW_STRIPS
#define LONG_ROW_STRIPS 2
#endif

namespace sffft {

constexpr int LC_COLS = 64;   // columns of a wavefront in the column passes (four 16-wide tiles)
constexpr int LC_WAVES = 4;   // wavefronts per workgroup in every pass
constexpr int LC_CBLOCK = LC_COLS * LC_WAVES;  // columns per column-pass workgroup

// w[v] = sc * exp(-2 pi i (e0 + step*v) / N), v = 0..3, N a power of two known at run
// time (inv_n = 1/N, exact): the base from v_sin/v_cos of the angle reduced to
// (-1/2, 1/2] revolutions, the others by a complex recurrence (as twiddle4e).
__device__ __forceinline__ void twiddle4_rt(int e0, int step, int N, float inv_n, float sc, float* wr, float* wi) {
  e0 &= N - 1;
  step &= N - 1;
  const float x0 = (float)(e0 > N / 2 ? e0 - N : e0) * inv_n;
  const float x1 = (float)(step > N / 2 ? step - N : step) * inv_n;
  float r = sc * cos_rev(x0), i = -sc * sin_rev(x0);
  const float sr = cos_rev(x1), si = -sin_rev(x1);
  wr[0] = r;
  wi[0] = i;
#pragma unroll
  for (int v = 1; v < 4; v++) {
    const float nr = r * sr - i * si, ni = r * si + i * sr;
    r = nr;
    i = ni;
    wr[v] = r;
    wi[v] = i;
  }
}

// Four complex fp16 points (re | im << 16 per dword) as an operand fragment: slots 0..3
// the real parts, 4..7 the imaginary parts.
__device__ __forceinline__ h8 cplx_operand(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3) {
  const u32x4 v = {(d0 & 0xffffu) | (d1 << 16), (d2 & 0xffffu) | (d3 << 16), (d0 >> 16) | (d1 & 0xffff0000u),
                   (d2 >> 16) | (d3 & 0xffff0000u)};
  return __builtin_bit_cast(h8, v);
}

// (dr + i di) * (wr + i wi) for four values, as four complex fp16 points (16 bytes).
__device__ __forceinline__ u32x4 cmul_points(f4 dr, f4 di, const float* wr, const float* wi) {
  h8 o;
#pragma unroll
  for (int v = 0; v < 4; v++) {
    o[2 * v] = (_Float16)(dr[v] * wr[v] - di[v] * wi[v]);
    o[2 * v + 1] = (_Float16)(dr[v] * wi[v] + di[v] * wr[v]);
  }
  return __builtin_bit_cast(u32x4, o);
}

template <int NC>
__host__ __device__ constexpr float inv_sqrt_radix() {
  return NC == 16 ? 0.25f : NC == 32 ? 0.17677669529663688f : 0.125f;
}

// Column-pass geometry: workgroup blockIdx.x covers LC_CBLOCK columns of pair
// pi = pi0 + blockIdx.x / (NR / LC_CBLOCK), pi = h*(B/2) + bp (rows (2bp, h) and
// (2bp+1, h)); wavefront `wave` takes LC_COLS of them. A launch covers the pairs of one
// chunk of channels, from pair pi0 on; the workspace holds the chunk (slot pi - pi0).
struct ColBlock {
  int pi, slot, cb;
  size_t ra, rb;  // element offsets of the pair's two rows in u / y
};
__device__ __forceinline__ ColBlock col_block(int B, int H, int L, int NR, int pi0, int wave) {
  const int cblocks = NR / LC_CBLOCK;
  ColBlock c;
  c.slot = blockIdx.x / cblocks;
  c.pi = pi0 + c.slot;
  c.cb = ((blockIdx.x - c.slot * cblocks) * LC_WAVES + wave) * LC_COLS;
  const int BP = B >> 1, h = c.pi / BP, bp = c.pi - h * BP;
  c.ra = ((size_t)(2 * bp) * H + h) * L;
  c.rb = c.ra + (size_t)H * L;
  return c;
}

// ---- pass A: DFT over n1 (rows n1 < NC/2 only, or all with CIRC), N-level twiddle,
// T in fp16. Lane (r, g) of tile (mt, ks) holds x[n1 = 16ks + 4g + j][n2 = cb + 16mt + r]
// (slots j: row a, 4 + j: row b); the result tile D[m][k1] puts four consecutive columns
// of one k1 in a lane, stored as 16 contiguous bytes of T.
template <int NC, class TIO, bool CIRC>
__global__ void __launch_bounds__(64 * LC_WAVES)
    long_cols_fwd(const TIO* __restrict__ u, uint32_t* __restrict__ work, int B, int H, int NR, int pi0,
                  float inv_n, const h8* __restrict__ ftab) {
  constexpr int MT = LC_COLS / 16;
  constexpr int KS = CIRC ? NC / 16 : NC >= 32 ? NC / 32 : 1;  // K steps over the non-zero rows
  constexpr int KT = NC / 16;                                  // 16-wide tiles of k1
  constexpr bool SPLIT = sizeof(TIO) == 4;  // fp32 input as fp16 value + fp16 remainder
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int N = NC * NR, LEN = CIRC ? N : N / 2;  // row length of u and y
  const ColBlock cbk = col_block(B, H, LEN, NR, pi0, wave);
  // The wavefront's block, rows n1 < NZ of both sequences and LC_COLS columns, is read
  // as 16-byte row chunks (whole 128-byte lines, CPR lanes per row), every load issued
  // before the first is used; then, one K step at a time, the chunks go through the
  // wavefront's LDS scratch into the operand layout (lane (r, g): column 16mt + r, rows
  // 16ks + 4g + j). The scratch rows are 16 bytes longer than the block, which puts the
  // four lane groups' rows on different banks.
  constexpr int NZ = CIRC ? NC : NC / 2;  // non-zero rows n1 (the rest is the zero padding)
  constexpr int KR = NZ < 16 ? NZ : 16;   // non-zero rows per K step and sequence
  constexpr int EPC = 16 / (int)sizeof(TIO), CPR = LC_COLS / EPC, PITCH = LC_COLS + EPC;
  constexpr int LPK = 2 * KR * CPR / 64;  // load instructions per K step
  static_assert(2 * KR * CPR % 64 == 0 && KS * KR == NZ, "whole load rounds per K step");
  __shared__ __attribute__((aligned(16))) TIO scratch[LC_WAVES][2 * KR * PITCH];
  TIO* S = scratch[wave];
  u32x4 c[KS][LPK];
#pragma unroll
  for (int ks = 0; ks < KS; ks++)
#pragma unroll
    for (int i = 0; i < LPK; i++) {
      const int q = i * 64 + lane, row = q / CPR, seq = row / KR;
      const size_t off = (size_t)(16 * ks + row - seq * KR) * NR + cbk.cb + (q % CPR) * EPC;
      c[ks][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(u + (seq ? cbk.rb : cbk.ra) + off));
    }
  h8 ah[MT][KS], al[SPLIT ? MT : 1][KS];
#pragma unroll
  for (int ks = 0; ks < KS; ks++) {
#pragma unroll
    for (int i = 0; i < LPK; i++) {
      const int q = i * 64 + lane;
      *reinterpret_cast<u32x4*>(S + (q / CPR) * PITCH + (q % CPR) * EPC) = c[ks][i];
    }
    wave_lds_fence();  // other lanes' chunks are read below
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int row = 4 * g + (j & 3);
        const float x = row < KR ? io_to_f32(S[((j < 4 ? 0 : KR) + row) * PITCH + 16 * mt + r]) : 0.f;
        const _Float16 hi = (_Float16)x;
        ah[mt][ks][j] = hi;
        if constexpr (SPLIT) al[mt][ks][j] = (_Float16)(x - (float)hi);
      }
    wave_lds_fence();  // every lane has read the block before the next K step overwrites it
  }

  uint32_t* T = work + (size_t)cbk.slot * N;
#pragma unroll
  for (int kt = 0; kt < KT; kt++) {
    h8 f0[KS], f1[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
      f0[ks] = cf_frag<NC, true>(ftab, kt, ks, 0, lane);
      f1[ks] = cf_frag<NC, true>(ftab, kt, ks, 1, lane);
    }
    const int k1 = 16 * kt + r;
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
      f4 dr = {0.f, 0.f, 0.f, 0.f}, di = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ks++) {
        dr = mfma(ah[mt][ks], f0[ks], dr);
        di = mfma(ah[mt][ks], f1[ks], di);
        if constexpr (SPLIT) {
          dr = mfma(al[mt][ks], f0[ks], dr);
          di = mfma(al[mt][ks], f1[ks], di);
        }
      }
      const int n2 = cbk.cb + 16 * mt + 4 * g;
      float wr[4], wi[4];
      twiddle4_rt(k1 * n2, k1, N, inv_n, inv_sqrt_radix<NC>(), wr, wi);
      *reinterpret_cast<u32x4*>(T + (size_t)k1 * NR + n2) = cmul_points(dr, di, wr, wi);
    }
  }
}

// ---- pass B: one row k1 of one pair per wavefront ---------------------------------
// Row order ((c*NC + k1)*BP + bp) over the channels h = h0 + c of the chunk: the B/2 rows
// that read one spectrum row are adjacent and run in the same workgroup. The workgroup copies the DFT fragments (first kind
// only; the second is derived in registers, dft_frag<R, true>) and the row plan's
// twiddle tables into LDS once, then its wavefronts loop over rows.
template <int R0, int R1>
struct LongRowPlan {
  typedef WavePlan<R0, R1> P;
  static constexpr int NR = R0 * R1;
  static constexpr int F0_H8 = P::F0_H8 / 2, F1_H8 = P::F1_H8 / 2;
  static constexpr int TAB_F4 = F0_H8 + F1_H8 + P::TW_TABLES * P::TW_F4;
  static constexpr int LDS_BYTES = TAB_F4 * 16;
  static_assert(LDS_BYTES <= 163840, "tables fit the LDS");
};

template <int R0, int R1>
__device__ __forceinline__ void long_row(uint32_t* x, const float4* __restrict__ SP, int k1, int N, float inv_n,
                                         float sc, const h8* F0, const h8* F1, const float4* TW1,
                                         const float4* TW2, int lane) {
  typedef WavePlan<R0, R1> P;
  constexpr int M = P::M, MT = P::MT, ST = P::ST, KF = R0 / 16;
  constexpr bool TWS = false;  // paired twiddle layout (tw_index): the split one measured 0.5-0.8% slower here
  const int r = lane & 15, g = lane >> 4;
  // compiler-only barrier at the top of each tile step: keeps the next step's table and
  // spectrum reads from being hoisted over the current one (all of them at once would
  // not fit beside the row)
  auto step_fence = [] { __asm__ volatile("" ::: "memory"); };

  // the whole row: lane (r, g) of tile (mt, ks) holds n2 = (16ks + 4g + j)*M + 16mt + r
  uint32_t raw[MT][KF][4];
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int ks = 0; ks < KF; ks++)
#pragma unroll
      for (int j = 0; j < 4; j++) raw[mt][ks][j] = x[(16 * ks + 4 * g + j) * M + 16 * mt + r];

  // ---- phase 1: DFT over n0 (all R0 rows), twiddle -> B2[m tile][k0 strip]. One m tile
  // at a time, so its input dies before the next tile's results are made.
  h8 b2[MT][ST];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) {
    h8 a[KF];
#pragma unroll
    for (int ks = 0; ks < KF; ks++)
      a[ks] = cplx_operand(raw[mt][ks][0], raw[mt][ks][1], raw[mt][ks][2], raw[mt][ks][3]);
#pragma unroll
    for (int nt = 0; nt < ST; nt++) {
      step_fence();
      f4 dr = {0.f, 0.f, 0.f, 0.f}, di = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KF; ks++) {
        dr = mfma(a[ks], dft_frag<R0, true>(F0, nt, ks, 0, lane), dr);
        di = mfma(a[ks], dft_frag<R0, true>(F0, nt, ks, 1, lane), di);
      }
      const int t = mt * ST + nt;
      b2[mt][nt] = cmul_pack(dr, di, TW1[tw_index(TWS, t, lane, 0)], TW1[tw_index(TWS, t, lane, 1)]);
    }
  }

  // ---- phase 2: per k0 strip, DFT over n1, spectrum, inverse DFT over k1, twiddle.
  // Strips are taken SG at a time, so that each DFT fragment read from LDS (and its
  // second kind rebuilt in registers) serves SG strips; the accumulation order of every
  // output is the same for any SG.
  constexpr int SG = ST % LONG_ROW_STRIPS == 0 ? LONG_ROW_STRIPS : 1;
#pragma unroll
  for (int s0 = 0; s0 < ST; s0 += SG) {
    h8 a2[SG][MT];
#pragma unroll
    for (int kt = 0; kt < MT; kt++) {
      step_fence();
      f4 dr[SG], di[SG];
#pragma unroll
      for (int j = 0; j < SG; j++) dr[j] = di[j] = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int mt = 0; mt < MT; mt++) {
        const h8 fa = dft_frag<R1, true>(F1, kt, mt, 0, lane), fb = dft_frag<R1, true>(F1, kt, mt, 1, lane);
#pragma unroll
        for (int j = 0; j < SG; j++) {
          dr[j] = mfma(fa, b2[mt][s0 + j], dr[j]);
          di[j] = mfma(fb, b2[mt][s0 + j], di[j]);
        }
      }
#pragma unroll
      for (int j = 0; j < SG; j++) {
        const int tile = (s0 + j) * MT + kt;
        a2[j][kt] = spectrum_conj_pack(dr[j], di[j], SP[sp_index(tile, lane, 0)], SP[sp_index(tile, lane, 1)]);
      }
    }
#pragma unroll
    for (int t = 0; t < MT; t++) {
      step_fence();
      f4 er[SG], ei[SG];
#pragma unroll
      for (int j = 0; j < SG; j++) er[j] = ei[j] = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kt = 0; kt < MT; kt++) {
        const h8 fa = dft_frag<R1, true>(F1, t, kt, 0, lane), fb = dft_frag<R1, true>(F1, t, kt, 1, lane);
#pragma unroll
        for (int j = 0; j < SG; j++) {
          er[j] = mfma(a2[j][kt], fa, er[j]);
          ei[j] = mfma(a2[j][kt], fb, ei[j]);
        }
      }
#pragma unroll
      for (int j = 0; j < SG; j++) {
        const int tt = (s0 + j) * MT + t;
        b2[t][s0 + j] = cmul_pack(er[j], ei[j], TW2[tw_index(TWS, tt, lane, 0)], TW2[tw_index(TWS, tt, lane, 1)]);
      }
    }
  }

  // ---- phase 3: DFT over k0 for all R0 rows n0; lane (c, g) of tile (nu, t) holds
  // n2 = (16nu + c)*M + 16t + 4g + v: times w_N^(n2 k1) sc, stored in place (16 bytes)
#pragma unroll
  for (int nu = 0; nu < ST; nu++) {
    step_fence();
    h8 f0[ST], f1[ST];
#pragma unroll
    for (int s = 0; s < ST; s++) {
      f0[s] = dft_frag<R0, true>(F0, nu, s, 0, lane);
      f1[s] = dft_frag<R0, true>(F0, nu, s, 1, lane);
    }
#pragma unroll
    for (int t = 0; t < MT; t++) {
      f4 zr = {0.f, 0.f, 0.f, 0.f}, zi = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < ST; s++) {
        zr = mfma(b2[t][s], f0[s], zr);
        zi = mfma(b2[t][s], f1[s], zi);
      }
      const int n2 = (16 * nu + r) * M + 16 * t + 4 * g;
      float wr[4], wi[4];
      twiddle4_rt(k1 * n2, k1, N, inv_n, sc, wr, wi);
      *reinterpret_cast<u32x4*>(x + n2) = cmul_points(zr, zi, wr, wi);
    }
  }
}

template <int R0, int R1>
__global__ void __launch_bounds__(64 * LC_WAVES)
    long_rows(uint32_t* work, const float4* __restrict__ kf, int nrows, int BP, int NC, int h0, float inv_n,
              float sc, const h8* __restrict__ ftab, const float4* __restrict__ twtab) {
  typedef WavePlan<R0, R1> P;
  typedef LongRowPlan<R0, R1> Q;
  constexpr int NR = Q::NR;
  const int N = NC * NR;
  __shared__ float4 lds[Q::TAB_F4];
  h8* F0 = reinterpret_cast<h8*>(lds);
  h8* F1 = R1 == R0 ? F0 : F0 + Q::F0_H8;
  float4* TW1 = lds + Q::F0_H8 + Q::F1_H8;
  float4* TW2 = P::TW_TABLES == 2 ? TW1 + P::TW_F4 : TW1;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // first-kind runs of the coefficient table: LDS run i is table run 2i
  auto tab = [&](int R, int k) { return reinterpret_cast<const float4*>(ftab + cf_off(R) + ((k >> 6) << 7) + (k & 63)); };
  dma_to_lds<P::TW_TABLES * P::TW_F4, LC_WAVES>(TW1, [&](int k) { return twtab + k; }, lane, wave);
  dma_to_lds<Q::F0_H8, LC_WAVES>(reinterpret_cast<float4*>(F0), [&](int k) { return tab(R0, k); }, lane, wave);
  if constexpr (R1 != R0)
    dma_to_lds<Q::F1_H8, LC_WAVES>(reinterpret_cast<float4*>(F1), [&](int k) { return tab(R1, k); }, lane, wave);
  wait_vmcnt<0>();
  __syncthreads();

  for (int row = blockIdx.x * LC_WAVES + wave; row < nrows; row += gridDim.x * LC_WAVES) {
    // compiler-only barrier: keeps the table reads of one row from being hoisted into
    // the previous one (they would stay live across it)
    __asm__ volatile("" ::: "memory");
    const int ck = row / BP, bp = row - ck * BP;  // ck = c*NC + k1
    const int c = ck / NC, k1 = ck - c * NC;
    uint32_t* x = work + ((size_t)(c * BP + bp) * NC + k1) * NR;
    const size_t hk = (size_t)(h0 + c) * NC + k1;  // the spectrum row
    long_row<R0, R1>(x, kf + hk * (NR / 2), k1, N, inv_n, sc, F0, F1, TW1, TW2, lane);
  }
}

// ---- pass C: DFT over k1 (all NC rows of U), outputs n1 < NC/2 (all with CIRC) --------
template <int NC, class TIO, bool CIRC>
__global__ void __launch_bounds__(64 * LC_WAVES)
    long_cols_inv(const uint32_t* __restrict__ work, TIO* __restrict__ y, int B, int H, int NR, int pi0,
                  const h8* __restrict__ ftab) {
  constexpr int MT = LC_COLS / 16;
  constexpr int KS = NC / 16;                                  // K steps over all k1
  constexpr int NT = CIRC ? NC / 16 : NC >= 32 ? NC / 32 : 1;  // result tiles of the stored n1
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int N = NC * NR, LEN = CIRC ? N : N / 2;
  const ColBlock cbk = col_block(B, H, LEN, NR, pi0, wave);
  const uint32_t* U = work + (size_t)cbk.slot * N;

  uint32_t raw[MT][KS][4];
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int ks = 0; ks < KS; ks++)
#pragma unroll
      for (int j = 0; j < 4; j++) raw[mt][ks][j] = U[(size_t)(16 * ks + 4 * g + j) * NR + cbk.cb + 16 * mt + r];
  h8 a[MT][KS];
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int ks = 0; ks < KS; ks++)
      a[mt][ks] = cplx_operand(raw[mt][ks][0], raw[mt][ks][1], raw[mt][ks][2], raw[mt][ks][3]);

#pragma unroll
  for (int nu = 0; nu < NT; nu++) {
    h8 f0[KS], f1[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
      f0[ks] = cf_frag<NC, true>(ftab, nu, ks, 0, lane);
      f1[ks] = cf_frag<NC, true>(ftab, nu, ks, 1, lane);
    }
    const int n1 = 16 * nu + r;
    const bool out = CIRC || NC >= 32 || n1 < NC / 2;
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
      f4 dr = {0.f, 0.f, 0.f, 0.f}, di = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ks++) {
        dr = mfma(a[mt][ks], f0[ks], dr);
        di = mfma(a[mt][ks], f1[ks], di);
      }
      const size_t off = (size_t)n1 * NR + cbk.cb + 16 * mt + 4 * g;
      if (out) {
        put4(y + cbk.ra + off, dr);
        put4(y + cbk.rb + off, -di);  // row b is minus the imaginary part
      }
    }
  }
}

}  // namespace sffft
