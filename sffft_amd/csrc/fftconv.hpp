// Fused causal long convolution for AMD Instinct MI355X (gfx950, CDNA4).
//
//   y[b,h,n] = sum_{m<=n} u[b,h,m] * k[h,n-m],   n < L
//
// computed as a length N = 2L transform, N = R0*R1(*R2), radices 16/32/64,
// in ONE launch per batch, one workgroup per sequence (NSEQ=1) or per pair of
// sequences of the same channel packed as the real and imaginary parts of one
// complex transform (NSEQ=2). Everything between the input load and the output
// store stays in LDS and VGPRs.
//
// Reference behaviour followed (file:line in the reference tree):
//   plan geometry ............. src/sffft.cu:92-104  (Plan<R0,R1,R2>)
//   twiddle exponent .......... src/sffft.cu:106-113 (twid<P,J>)
//   stage schedule ............ src/sffft.cu:273-279 (L0f [L1f] Rf Ri [L1i] L0i)
//   real-input / real-output .. src/sffft.cu:142-144,164-165,180-181
//   spectrum fused between the last forward and first inverse stage:
//                               src/sffft.cu:229-236
//   fp16 storage, fp32 twiddle/spectrum arithmetic: src/sffft.cu:120-135
//
// MI355X design (not a translation of the WMMA code):
//  * Every stage is a dense complex contraction on v_mfma_f32_16x16x32_f16.
//    A complex K=16 contraction is one real K=32 contraction: operand slots
//    0..3 of lane (i, g=lane/16) hold the real parts of complex index 4g..4g+3,
//    slots 4..7 the imaginary parts, so Dr = [Xr|Xi].[Fr;-Fi] and
//    Di = [Xr|Xi].[Fi;Fr] are two MFMAs per 16-wide complex K step.
//  * The MFMA D layout (lane (c,g) holds rows 4g..4g+3 of column c) equals the
//    A/B operand layout of the next contraction over those rows, so chained
//    contractions stay in registers: in two-stage plans the last forward stage,
//    the spectrum product and the first inverse stage; in three-stage plans all
//    four stages of a k0 row (phase 2), whose input alone comes from LDS.
//  * Between phases the LDS layout changes so the next contraction digit is the
//    fastest one: operand reads and accumulator writes are 8-byte vectors, and
//    XOR swizzles keep the remaining scalar writes off shared banks.
//  * Inverse stages reuse the forward DFT fragments: IDFT(X) = conj(DFT(conj X));
//    the conjugations are folded into the twiddle and spectrum products.
//  * Twiddles are computed in registers with v_sin_f32/v_cos_f32 (argument in
//    revolutions, so e/N is exact) and a 3-step complex recurrence; with eight
//    rows per wavefront, the last twiddles of phase 2 step from row to row.
//  * fp32 I/O: the input enters the first stage as an fp16 value plus its fp16
//    remainder (SFFFT_FP32_SPLITS), removing the largest rounding term.
#pragma once
#include <hip/hip_runtime.h>

#include <type_traits>
#include <stdint.h>

// fp16 operands of fp32-I/O three-stage plans that also carry their fp16 remainder
// (x = hi + lo, the contraction run on both: ~22 significant bits instead of 11, for
// twice that contraction's MFMAs). Bit 3: the input of the first stage; bits 0, 1, 2:
// the operands of the stage over n2, the inverse over k2 (the spectrum product) and the
// inverse over k1. Measured at B=8 H=768 with pairs of sequences per transform: the
// input split (8) takes rel-L2 from 4.7e-4..5.1e-4 to 4.2e-4..4.7e-4 for 3-5% time;
// all four (15) reach 3.3e-4..3.7e-4 for 22-41%.
#ifndef SFFFT_FP32_SPLITS
#define SFFFT_FP32_SPLITS 8
#endif

// k0 rows per phase-2 step of three-stage plans (each wavefront's rows taken this many at a time)
#ifndef SFFFT_WG_ROWS
#define SFFFT_WG_ROWS 4
#endif

namespace sffft {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int LDS_PAD = 4;  // halves appended to each LDS row (keeps 8-byte alignment)

// DFT fragment table (units of h8 = one lane's 8 halves; 64 lanes per fragment).
//   CF[R][a][b][kind]: complex fragments, lane (r,g), slot v<4:
//        kind 0: [ cos t | sin t ],  kind 1: [ -sin t | cos t ],
//        t = 2*pi*((16a+r)*(16b+4g+v) mod R)/R  (F = exp(-i t) is symmetric)
//   RI[R][nt][kind]: real-input fragments (one sequence), lane (c,g), slot j:
//        n0 = j<4 ? 4g+j : 16+4g+(j-4),  t = 2*pi*((n0*(16nt+c)) mod R)/R
//        kind 0: cos t, kind 1: -sin t;  zero for n0 >= R/2 (the zero-padded half)
__host__ __device__ constexpr int cf_off(int R) { return R == 16 ? 0 : R == 32 ? 256 : 1024; }
__host__ __device__ constexpr int ri_off(int R) { return R == 16 ? 128 : R == 32 ? 768 : 3072; }
constexpr int FTAB_H8 = 3584;

__host__ __device__ constexpr int cmax(int a, int b) { return a > b ? a : b; }

template <int R0_, int R1_, int R2_ = 1>
struct Plan {
  static constexpr int R0 = R0_, R1 = R1_, R2 = R2_;
  static constexpr int S = R2_ > 1 ? 3 : 2;
  static constexpr int N = R0 * R1 * R2, L = N / 2;
  static constexpr int M = N / R0;           // positions per first-digit row
  static constexpr int PA = R1 + LDS_PAD;    // pitch: rows whose fastest digit is n1/k1
  static constexpr int PB = R0 + LDS_PAD;    // pitch: [m][k0], input of the last inverse stage (two-stage)
  static constexpr int ROW = S == 3 ? R2 * PA : 0;  // one k0 row of [k0][n2][n1] (three-stage)
  static constexpr int PLANE0 = S == 3 ? R0 * ROW : cmax(R0 * PA, R1 * PB);
  static constexpr int PLANE = (PLANE0 + 63) & ~63;
  static constexpr int LDS_BYTES = 2 * PLANE * 2;
  static_assert(R0 >= 16 && R1 >= 16 && (S == 2 || R2 >= 16), "radices are 16, 32 or 64");
  static_assert(R0 <= 64 && R1 <= 64 && R2 <= 64, "radices are 16, 32 or 64");
};

__device__ __forceinline__ f4 mfma(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float sin_rev(float x) { return __builtin_amdgcn_sinf(x); }  // sin(2*pi*x)
__device__ __forceinline__ float cos_rev(float x) { return __builtin_amdgcn_cosf(x); }  // cos(2*pi*x)

// ---- I/O element conversions -------------------------------------------------
__device__ __forceinline__ float io_to_f32(float x) { return x; }
__device__ __forceinline__ float io_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
// fp32 -> bf16, IEEE round-to-nearest-even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t x = __float_as_uint(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// Four fp32 values as four bf16 in two dwords, round to nearest even: the gfx950
// packed conversion, two values per instruction (f32_to_bf16 costs six per value).
__device__ __forceinline__ u32x2 f4_to_bf16x4(f4 v) {
  typedef float fl2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  const bf2 lo = __builtin_convertvector((fl2){v[0], v[1]}, bf2);
  const bf2 hi = __builtin_convertvector((fl2){v[2], v[3]}, bf2);
  return (u32x2){__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
}
// fp16-accumulation mode: the raw tile accumulator is rounded to fp16 (range and
// rounding of an fp16 accumulator; +-inf beyond 65504).
__device__ __forceinline__ f4 round_acc(f4 v, int acc16) {
  if (acc16) {
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = (float)(_Float16)v[i];
  }
  return v;
}

// -1 in a register the compiler cannot see through: fma(-1, (float)h, x) with a known
// -1 becomes x - (float)h, three instructions (convert, subtract, convert) instead of
// one mixed-precision fma.
__device__ __forceinline__ float minus_one() {
  float m = -1.f;
  asm volatile("" : "+v"(m));
  return m;
}

// ---- DFT fragments ------------------------------------------------------------
template <int R, bool CACHED>
__device__ __forceinline__ h8 cf_frag(const h8* __restrict__ ftab, int a, int b, int kind, int lane) {
  if constexpr (CACHED) {
    return ftab[cf_off(R) + ((a * (R / 16) + b) * 2 + kind) * 64 + lane];
  } else {
    const int r = lane & 15, g = lane >> 4;
    h8 f;
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int e = ((16 * a + r) * (16 * b + 4 * g + v)) & (R - 1);
      const float x = (float)e * (1.0f / R);
      const _Float16 s = (_Float16)sin_rev(x), c = (_Float16)cos_rev(x);
      f[v] = kind == 0 ? c : -s;
      f[4 + v] = kind == 0 ? s : c;
    }
    return f;
  }
}
template <int R, bool CACHED>
__device__ __forceinline__ h8 ri_frag(const h8* __restrict__ ftab, int nt, int kind, int lane) {
  if constexpr (CACHED) {
    return ftab[ri_off(R) + (nt * 2 + kind) * 64 + lane];
  } else {
    const int c = lane & 15, g = lane >> 4;
    h8 f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int n0 = j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4);
      const int e = (n0 * (16 * nt + c)) & (R - 1);
      const float x = (float)e * (1.0f / R);
      f[j] = n0 >= R / 2 ? (_Float16)0.f : kind == 0 ? (_Float16)cos_rev(x) : -(_Float16)sin_rev(x);
    }
    return f;
  }
}

// The complex DFT fragments of radix R for a loop over rows: evaluated once and held
// in registers (HOLD), or produced at each use. Held fragments pass through an empty
// asm so the compiler neither re-evaluates them per row nor sinks them into the loop.
template <int R, bool CACHED, bool HOLD>
struct FragSet {
  static constexpr int T = HOLD ? R / 16 : 1;
  h8 f[T][T][2];
  __device__ __forceinline__ void init(const h8* __restrict__ ftab, int lane) {
    if constexpr (HOLD) {
#pragma unroll
      for (int a = 0; a < T; a++)
#pragma unroll
        for (int b = 0; b < T; b++)
#pragma unroll
          for (int k = 0; k < 2; k++) {
            f[a][b][k] = cf_frag<R, CACHED>(ftab, a, b, k, lane);
            asm volatile("" : "+v"(f[a][b][k]));
          }
    }
  }
  __device__ __forceinline__ h8 get(const h8* __restrict__ ftab, int a, int b, int kind, int lane) const {
    if constexpr (HOLD) return f[a][b][kind];
    else return cf_frag<R, CACHED>(ftab, a, b, kind, lane);
  }
};

// w[v] = sc * exp(-2*pi*i * (e0 + step*v) / N), v = 0..3 (src/sffft.cu:106-113 for the
// exponent): the base from v_sin/v_cos with the angle reduced to (-1/2, 1/2]
// revolutions (e/N is exact), the others by a complex recurrence.
template <int N>
__device__ __forceinline__ void twiddle4e(int e0, int step, float sc, float* wr, float* wi) {
  e0 &= N - 1;
  step &= N - 1;
  const float x0 = (float)(e0 > N / 2 ? e0 - N : e0) * (1.0f / N);
  const float x1 = (float)(step > N / 2 ? step - N : step) * (1.0f / N);
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
// (r, i) *= (fr, fi), four values
__device__ __forceinline__ void cmul4(float* r, float* i, const float* fr, const float* fi) {
#pragma unroll
  for (int v = 0; v < 4; v++) {
    const float nr = r[v] * fr[v] - i[v] * fi[v], ni = r[v] * fi[v] + i[v] * fr[v];
    r[v] = nr;
    i[v] = ni;
  }
}
// w[v] = sc * exp(-2*pi*i * a*(b0+v) / N)
template <int N>
__device__ __forceinline__ void twiddle4(int a, int b0, float sc, float* wr, float* wi) {
  twiddle4e<N>(a * b0, a, sc, wr, wi);
}

// 8-half operand: slots 0..3 from the real plane, 4..7 from the imaginary plane.
// Orders one wavefront's LDS accesses across its lanes (a lane reads what other lanes
// of the same wavefront wrote, or overwrites what they read). A wavefront's LDS
// operations complete in issue order, so the product build needs only a compiler
// barrier: the compiler models each lane alone and would otherwise reuse a lane's
// earlier reads or move writes above reads. The SFFFT_DEBUG_BARRIERS build also waits
// until every LDS operation of the wavefront has completed, so it cannot depend on the
// in-order completion; its outputs are compared bit for bit with the product build's.
__device__ __forceinline__ void wave_lds_fence() {
#ifdef SFFFT_DEBUG_BARRIERS
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __builtin_amdgcn_wave_barrier();
#endif
  __asm__ volatile("" ::: "memory");
}

// The same wait in the SFFFT_DEBUG_BARRIERS build only, where the product build relies
// on program order alone (a wavefront overwriting LDS its lanes have read).
__device__ __forceinline__ void debug_lds_fence() {
#ifdef SFFFT_DEBUG_BARRIERS
  wave_lds_fence();
#endif
}

__device__ __forceinline__ h8 lds_frag(const _Float16* re, const _Float16* im, int pos) {
  const h4 a = *reinterpret_cast<const h4*>(re + pos);
  const h4 b = *reinterpret_cast<const h4*>(im + pos);
  return (h8){a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}
__device__ __forceinline__ h4 to_h4(const float* x) {
  return (h4){(_Float16)x[0], (_Float16)x[1], (_Float16)x[2], (_Float16)x[3]};
}

// ---- Products of the fp16-accumulation mode -------------------------------------
// The mode rounds every accumulator to fp16 (the reference's fp16 accumulators,
// src/sffft.cu:88,397-398). Its twiddle and spectrum products then run in packed fp16 on
// those rounded values: v_cvt_pk_f16_f32 (the rounding itself), v_pk_mul_f16 and
// v_pk_fma_f16, two values per instruction, instead of the fp32 products and separate
// roundings of fp32 accumulation: the speed-for-precision trade of that mode
// (README.md:112-122).
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ h2 pk_h2(float a, float b) { return __builtin_convertvector((f2){a, b}, h2); }
// four complex factors in packed fp16
struct HW {
  h2 r01, r23, i01, i23;
};
__device__ __forceinline__ HW hw_of(const float* wr, const float* wi) {
  return HW{pk_h2(wr[0], wr[1]), pk_h2(wr[2], wr[3]), pk_h2(wi[0], wi[1]), pk_h2(wi[2], wi[3])};
}
// (dr + i di) w for four values, as fp16 real parts xr and imaginary parts xi (CONJ: the
// conjugate of the product)
template <bool CONJ = false>
__device__ __forceinline__ void cmul_hp(f4 dr, f4 di, const HW& w, h4& xr, h4& xi) {
  const h2 r01 = pk_h2(dr[0], dr[1]), r23 = pk_h2(dr[2], dr[3]);
  const h2 i01 = pk_h2(di[0], di[1]), i23 = pk_h2(di[2], di[3]);
  const h2 a = r01 * w.r01 - i01 * w.i01, b = r23 * w.r23 - i23 * w.i23;
  h2 c, d;
  if constexpr (CONJ) {
    c = -(r01 * w.i01) - i01 * w.r01;
    d = -(r23 * w.i23) - i23 * w.r23;
  } else {
    c = r01 * w.i01 + i01 * w.r01;
    d = r23 * w.i23 + i23 * w.r23;
  }
  xr = (h4){a[0], a[1], b[0], b[1]};
  xi = (h4){c[0], c[1], d[0], d[1]};
}
__device__ __forceinline__ h8 join_h8(h4 a, h4 b) { return (h8){a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]}; }

// ---- Phase 1: first forward stage over n0 (src/sffft.cu:266-274) ---------------
// Input rows are natural order, n = n0*M + m. Data is the A operand (M = 16
// consecutive m, K = n0); only n0 < R0/2 is loaded (the zero-padded half is
// skipped). Output D[m][k0] is twiddled by w^(k0*m) and written with m fastest.
// Work split: the A tiles (16 consecutive m) are spread over the waves; when there
// are fewer A tiles than waves, the waves sharing a tile split its k0 tiles, so
// every input element is loaded by exactly one wave.
template <class P, int NW, int NSEQ>
struct P1Split {
  static constexpr int MT = P::M / 16, NT = P::R0 / 16;
  static constexpr bool BY_MT = MT >= NW;
  static constexpr int TPW = BY_MT ? MT / NW : 1;                // A tiles per wave
  static constexpr int WPM = BY_MT ? 1 : NW / MT;                // waves sharing one A tile
  static constexpr int NTW = BY_MT ? NT : (NT + WPM - 1) / WPM;  // k0 tiles per A tile and wave
  static constexpr int KS = NSEQ == 2 ? (P::R0 / 2 + 15) / 16 : 1;  // K steps
  __device__ static int mt(int wave, int i) { return BY_MT ? wave + i * NW : wave % MT; }
  __device__ static int nt(int wave, int j) { return BY_MT ? j : wave / MT + j * WPM; }
};

// The raw input elements of this wave's phase-1 A tiles: lane (r, g) of tile i holds
// row m = 16 mt + r at the 8 (NSEQ = 1) or 4 + 4 (NSEQ = 2) first-digit positions n0 of
// its K slots; positions in the zero-padded half (n0 >= R0/2) are not loaded.
template <class P, int NW, int NSEQ, class TIO>
struct P1Data {
  TIO raw[P1Split<P, NW, NSEQ>::TPW][P1Split<P, NW, NSEQ>::KS][8];
};

template <class P, int NSEQ>
__device__ __forceinline__ int p1_n0(int ks, int g, int j) {
  if constexpr (NSEQ == 2) return 16 * ks + 4 * g + (j & 3);
  else return j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4);
}

// Issues every input load of this wave's phase-1 tiles (one HBM round trip). The
// elements stay raw until their tile is computed, and the compiler barrier keeps all
// loads ahead of the first tile: converted here, or sunk to their use, the later
// tiles' loads would be issued only after the first tile's have landed.
template <class P, int NW, int NSEQ, class TIO>
__device__ __forceinline__ void p1_prefetch(const TIO* __restrict__ xa, const TIO* __restrict__ xb,
                                            P1Data<P, NW, NSEQ, TIO>& d, int lane, int wave) {
  using SP = P1Split<P, NW, NSEQ>;
  constexpr int R0 = P::R0, M = P::M;
  const int r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int i = 0; i < SP::TPW; i++) {
    const int m = 16 * SP::mt(wave, i) + r;
#pragma unroll
    for (int ks = 0; ks < SP::KS; ks++)
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int n0 = p1_n0<P, NSEQ>(ks, g, j);
        const TIO* src = NSEQ == 2 && j >= 4 ? xb : xa;
        d.raw[i][ks][j] = n0 < R0 / 2 ? src[n0 * M + m] : TIO(0);
      }
  }
  asm volatile("" ::: "memory");
}

// SPLIT_IN: the fp32 input enters the first stage as fp16 value plus fp16 remainder
// (twice that stage's MFMAs), so it is not rounded to 11 bits there.
// The first stage's DFT fragments of the wavefront's k0 tiles, read before the input so
// that waiting for them does not wait for the input. Used when a wavefront has at most
// two k0 tiles and at least four A tiles: measured 1.3-2% faster there (L = 8192 and
// 16384), 1-2% slower with two A tiles, where the registers cost occupancy.
template <class P, int NW, int NSEQ, bool CACHED>
struct P1Frags {
  using SP = P1Split<P, NW, NSEQ>;
  static constexpr int PF = SP::NTW <= 2 && SP::TPW >= 4 ? SP::NTW : 0;
  h8 f[PF > 0 ? PF : 1][SP::KS][2];
  __device__ __forceinline__ void load(const h8* __restrict__ ftab, int lane, int wave) {
    if constexpr (PF > 0) {
#pragma unroll
      for (int j = 0; j < PF; j++) {
        const int nt = SP::nt(wave, j);
        if (nt < SP::NT) {
#pragma unroll
          for (int ks = 0; ks < SP::KS; ks++)
#pragma unroll
            for (int k = 0; k < 2; k++)
              f[j][ks][k] = NSEQ == 2 ? cf_frag<P::R0, CACHED>(ftab, nt, ks, k, lane)
                                      : ri_frag<P::R0, CACHED>(ftab, nt, k, lane);
        }
      }
    }
  }
};

template <class P, int NW, int NSEQ, class TIO, bool CACHED, bool SPLIT_IN>
__device__ __forceinline__ void phase1(const P1Data<P, NW, NSEQ, TIO>& d, P1Frags<P, NW, NSEQ, CACHED>& fr,
                                       _Float16* re, _Float16* im, const h8* __restrict__ ftab, int acc16, int lane,
                                       int wave) {
  using SP = P1Split<P, NW, NSEQ>;
  constexpr int R0 = P::R0, N = P::N, KS = SP::KS, SI = SPLIT_IN ? 1 : 0;
  constexpr float sc0 = R0 == 16 ? 0.25f : R0 == 32 ? 0.17677669529663687f : 0.125f;
  const int r = lane & 15, g = lane >> 4;
  // Work that does not depend on the input is done while its HBM round trip is in
  // flight: the DFT fragments of the wavefront's k0 tiles (read before the input, see
  // P1Frags) and the first A tile's twiddles are made final (empty asms) before a
  // scheduling barrier that the first use of the input, where the wait for it lands,
  // cannot cross. Without them the compiler sinks both to their first use.
  constexpr int PF = P1Frags<P, NW, NSEQ, CACHED>::PF;
  float t0r[PF > 0 ? PF : 1][4], t0i[PF > 0 ? PF : 1][4];
  if constexpr (PF > 0) {
#pragma unroll
    for (int j = 0; j < PF; j++) {
      const int nt = SP::nt(wave, j);
      if (nt < SP::NT) {
#pragma unroll
        for (int ks = 0; ks < KS; ks++)
#pragma unroll
          for (int k = 0; k < 2; k++) asm volatile("" : "+v"(fr.f[j][ks][k]));
        twiddle4<N>(16 * nt + r, 16 * SP::mt(wave, 0) + 4 * g, sc0, t0r[j], t0i[j]);
#pragma unroll
        for (int v = 0; v < 4; v++) asm volatile("" : "+v"(t0r[j][v]), "+v"(t0i[j][v]));
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  auto frag = [&](int j, int nt, int ks, int k) {
    if constexpr (PF > 0) return fr.f[j][ks][k];
    else if constexpr (NSEQ == 2) return cf_frag<R0, CACHED>(ftab, nt, ks, k, lane);
    else return ri_frag<R0, CACHED>(ftab, nt, k, lane);
  };
#pragma unroll
  for (int i = 0; i < SP::TPW; i++) {
    const int mt = SP::mt(wave, i);
    h8 a[KS][1 + SI];
#pragma unroll
    for (int ks = 0; ks < KS; ks++)
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const float x = io_to_f32(d.raw[i][ks][j]);
        a[ks][0][j] = (_Float16)x;
        if constexpr (SPLIT_IN) a[ks][SI][j] = (_Float16)__builtin_fmaf(minus_one(), (float)a[ks][0][j], x);
      }
#pragma unroll
    for (int j = 0; j < SP::NTW; j++) {
      const int nt = SP::nt(wave, j);
      if (nt < SP::NT) {
        f4 dr = {0.f, 0.f, 0.f, 0.f}, di = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ks++)
#pragma unroll
          for (int p = 0; p <= SI; p++) {
            dr = mfma(a[ks][p], frag(j, nt, ks, 0), dr);
            di = mfma(a[ks][p], frag(j, nt, ks, 1), di);
          }
        const int k0 = 16 * nt + r;
        float wr[4], wi[4];
        if (PF > 0 && i == 0) {
#pragma unroll
          for (int v = 0; v < 4; v++) wr[v] = t0r[PF > 0 ? j : 0][v], wi[v] = t0i[PF > 0 ? j : 0][v];
        } else {
          twiddle4<N>(k0, 16 * mt + 4 * g, sc0, wr, wi);
        }
        h4 hr, hi;  // the twiddled tile in fp16
        if (acc16) {
          cmul_hp(dr, di, hw_of(wr, wi), hr, hi);
        } else {
          float xr[4], xi[4];
#pragma unroll
          for (int v = 0; v < 4; v++) {
            xr[v] = dr[v] * wr[v] - di[v] * wi[v];
            xi[v] = dr[v] * wi[v] + di[v] * wr[v];
          }
          hr = to_h4(xr);
          hi = to_h4(xi);
        }
        if constexpr (P::S == 2) {
          const int pos = k0 * P::PA + 16 * mt + 4 * g;  // [k0][n1]
          *reinterpret_cast<h4*>(re + pos) = hr;
          *reinterpret_cast<h4*>(im + pos) = hi;
        } else {
#pragma unroll
          for (int v = 0; v < 4; v++) {  // [k0][n2 ^ (k0 & 15)][n1]
            // The 16 lanes of this scalar write differ in k0, i.e. by whole ROW pitches
            // (multiples of the bank count): swizzling the row index with k0 spreads
            // them over 16 rows and banks. phase2_s3 reads the row back swizzled.
            const int m = 16 * mt + 4 * g + v, n1 = m / P::R2, n2 = m % P::R2;
            const int pos = k0 * P::ROW + (n2 ^ (k0 & 15)) * P::PA + n1;
            re[pos] = hr[v];
            im[pos] = hi[v];
          }
        }
      }
    }
  }
}

// ---- Spectrum product + first inverse stage (src/sffft.cu:229-236, 276-277) -----
// The spectrum tile of one lane: 4 complex64 values, rows 4g..4g+3 of column c of
// a 16x16 tile, stored contiguously in the kernel order (32 bytes per lane).
__device__ __forceinline__ void load_k4(const float2* __restrict__ kp, int lane, float4* q) {
  const float4* p = reinterpret_cast<const float4*>(kp + lane * 4);
  q[0] = p[0];
  q[1] = p[1];
}
// d = forward result tiles D[kk][c] (lane column c, rows 16*mt+4g+v), q = spectrum
// tiles. Returns A operands conj(D*K)^T for the inverse.
// With SPLIT, lo receives the fp16 remainders x - (float)hi: the inverse stage that
// follows runs on hi and on lo (twice the MFMAs of that stage), so the product enters
// it with about 22 significant bits instead of 11. One fp16 rounding of the five of a
// three-stage plan (three of a two-stage one) is removed this way.
// With acc16 (the fp16-accumulation mode) the raw accumulators are given and the product
// runs in packed fp16 (cmul_hp).
template <int T, bool SPLIT = false>
__device__ __forceinline__ void spectrum_product(const f4* dr, const f4* di, const float4 (*q)[2], h8* a2,
                                                 h8* lo = nullptr, int acc16 = 0) {
#pragma unroll
  for (int mt = 0; mt < T; mt++) {
    const float4 k01 = q[mt][0], k23 = q[mt][1];
    const float kr[4] = {k01.x, k01.z, k23.x, k23.z};
    const float ki[4] = {k01.y, k01.w, k23.y, k23.w};
    if (acc16) {
      h4 hr, hi;
      cmul_hp<true>(dr[mt], di[mt], hw_of(kr, ki), hr, hi);
      a2[mt] = join_h8(hr, hi);
      continue;
    }
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const float xr = dr[mt][v] * kr[v] - di[mt][v] * ki[v];
      const float xi = dr[mt][v] * ki[v] + di[mt][v] * kr[v];
      a2[mt][v] = (_Float16)xr;
      a2[mt][4 + v] = (_Float16)(-xi);
      if constexpr (SPLIT) {  // x - hi as one v_fma_mix each
        lo[mt][v] = (_Float16)__builtin_fmaf(minus_one(), (float)a2[mt][v], xr);
        lo[mt][4 + v] = (_Float16)__builtin_fmaf(minus_one(), (float)a2[mt][4 + v], -xi);
      }
    }
  }
}

// ---- Phase 2, two-stage plans: over n1, spectrum, inverse over k1 ----------------
template <class P, int NW>
struct KData2 {
  static constexpr int ST = P::R0 / 16, T1 = P::R1 / 16, UPW = (ST + NW - 1) / NW;
  float4 q[UPW][T1][2];
};

// Issues the spectrum loads of this wave's strips (kernel order, 1 KB per wave and tile).
template <class P, int NW>
__device__ __forceinline__ void k_prefetch_s2(const float2* __restrict__ K, KData2<P, NW>& d, int lane, int wave) {
  using D = KData2<P, NW>;
#pragma unroll
  for (int i = 0; i < D::UPW; i++) {
    const int s = wave + i * NW;
    if (s < D::ST) {
#pragma unroll
      for (int mt = 0; mt < D::T1; mt++) load_k4(K + (size_t)(s * D::T1 + mt) * 256, lane, d.q[i][mt]);
    }
  }
}

template <class P, int NW, bool CACHED, bool SPLIT>
__device__ __forceinline__ void phase2_s2(_Float16* re, _Float16* im, const KData2<P, NW>& kd,
                                          const h8* __restrict__ ftab, int acc16, int lane, int wave) {
  constexpr int R0 = P::R0, R1 = P::R1, N = P::N, ST = R0 / 16, T1 = R1 / 16;
  constexpr int UPW = (ST + NW - 1) / NW;
  constexpr float sc1 = R1 == 16 ? 0.25f : R1 == 32 ? 0.17677669529663687f : 0.125f;
  const int c = lane & 15, g = lane >> 4;
  h4 outr[UPW][T1], outi[UPW][T1];
#pragma unroll
  for (int i = 0; i < UPW; i++) {
    const int s = wave + i * NW;
    if (s < ST) {
      h8 b[T1];
#pragma unroll
      for (int ks = 0; ks < T1; ks++) b[ks] = lds_frag(re, im, (16 * s + c) * P::PA + 16 * ks + 4 * g);
      f4 dr[T1], di[T1];
#pragma unroll
      for (int mt = 0; mt < T1; mt++) {
        dr[mt] = (f4){0.f, 0.f, 0.f, 0.f};
        di[mt] = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < T1; ks++) {
          dr[mt] = mfma(cf_frag<R1, CACHED>(ftab, mt, ks, 0, lane), b[ks], dr[mt]);
          di[mt] = mfma(cf_frag<R1, CACHED>(ftab, mt, ks, 1, lane), b[ks], di[mt]);
        }
      }
      h8 a2[T1], a2lo[SPLIT ? T1 : 1];
      spectrum_product<T1, SPLIT>(dr, di, kd.q[i], a2, a2lo, acc16);
#pragma unroll
      for (int nt = 0; nt < T1; nt++) {
        f4 er = {0.f, 0.f, 0.f, 0.f}, ei = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int mt = 0; mt < T1; mt++) {
          er = mfma(a2[mt], cf_frag<R1, CACHED>(ftab, nt, mt, 0, lane), er);
          ei = mfma(a2[mt], cf_frag<R1, CACHED>(ftab, nt, mt, 1, lane), ei);
          if constexpr (SPLIT) {
            er = mfma(a2lo[mt], cf_frag<R1, CACHED>(ftab, nt, mt, 0, lane), er);
            ei = mfma(a2lo[mt], cf_frag<R1, CACHED>(ftab, nt, mt, 1, lane), ei);
          }
        }
        float wr[4], wi[4];
        twiddle4<N>(16 * nt + c, 16 * s + 4 * g, sc1, wr, wi);
        if (acc16) {
          cmul_hp(er, ei, hw_of(wr, wi), outr[i][nt], outi[i][nt]);
        } else {
          float xr[4], xi[4];
#pragma unroll
          for (int v = 0; v < 4; v++) {
            xr[v] = er[v] * wr[v] - ei[v] * wi[v];
            xi[v] = er[v] * wi[v] + ei[v] * wr[v];
          }
          outr[i][nt] = to_h4(xr);
          outi[i][nt] = to_h4(xi);
        }
      }
    }
  }
  __syncthreads();  // every strip has been read before the [n1][k0] layout is written
#pragma unroll
  for (int i = 0; i < UPW; i++) {
    const int s = wave + i * NW;
    if (s < ST) {
#pragma unroll
      for (int nt = 0; nt < T1; nt++) {
        const int pos = (16 * nt + c) * P::PB + 16 * s + 4 * g;
        *reinterpret_cast<h4*>(re + pos) = outr[i][nt];
        *reinterpret_cast<h4*>(im + pos) = outi[i][nt];
      }
    }
  }
}

// ---- Phase 2, three-stage plans: per k0 row, stages over n1 and n2, spectrum,
// inverse over k2 and k1 (src/sffft.cu:273-279). A row is owned by one wavefront and
// all its stages run in registers: the result tile of each contraction has the lane
// layout of the next one's B operand (lane (c, g) holds rows 4g..4g+3 of column c,
// and a B operand holds K indices 4g..4g+3 of column c):
//   stage over n1:  D[n2][k1]  = A[n2][n1] (LDS, [k0][n2][n1]) x F1,  then twiddle
//   stage over n2:  D2[k2][k1] = F2 x D          (D as B, K = n2)
//   spectrum:       A2[k1][k2] = conj(D2 K)^T    (the result lanes, read as A)
//   inverse k2:     E[n2][k1]^T = A2 x F2,  i.e. E[k1][n2] with n2 on the lane column;
//                   twiddle, then E as B (K = k1) of
//   inverse k1:     Z[n1][n2]  = F1 x E,  last twiddle w^(k0 m), m = n1 R2 + n2.
// Every operand is rounded to fp16 once. SPLITS (bits 0..2 of SFFFT_FP32_SPLITS for
// fp32 I/O) selects the operands made here in registers that also carry their fp16
// remainder, the contraction then running on both parts.
template <bool SPLIT>
__device__ __forceinline__ void pack_operand(const float* xr, const float* xi, h8& hi, h8& lo) {
#pragma unroll
  for (int v = 0; v < 4; v++) {
    hi[v] = (_Float16)xr[v];
    hi[4 + v] = (_Float16)xi[v];
    if constexpr (SPLIT) {  // x - hi as one v_fma_mix each (hi read as fp16, times -1)
      lo[v] = (_Float16)__builtin_fmaf(minus_one(), (float)hi[v], xr[v]);
      lo[4 + v] = (_Float16)__builtin_fmaf(minus_one(), (float)hi[4 + v], xi[v]);
    }
  }
}

template <class P, int NW, bool CACHED, int SPLITS>
__device__ __forceinline__ void phase2_s3(_Float16* re, _Float16* im, const float2* __restrict__ K,
                                          const h8* __restrict__ ftab, int acc16, int lane, int wave) {
  constexpr int R0 = P::R0, R1 = P::R1, R2 = P::R2, N = P::N, T1 = R1 / 16, T2 = R2 / 16;
  constexpr int ROWS = R0 / NW;
  constexpr int SB = SPLITS & 1, SE = (SPLITS >> 2) & 1;
  constexpr bool SA = (SPLITS >> 1) & 1;
  static_assert(R0 % NW == 0, "three-stage plans need R0 divisible by the wave count");
  constexpr float sc1 = R1 == 16 ? 0.25f : R1 == 32 ? 0.17677669529663687f : 0.125f;
  constexpr float sc2 = R2 == 16 ? 0.25f : R2 == 32 ? 0.17677669529663687f : 0.125f;
  const int c = lane & 15, g = lane >> 4;
  // In-kernel DFT fragments (legacy plans) are evaluated once for all rows when both
  // radices' sets fit in 40 VGPRs; table fragments are read at each use (holding them
  // measured no faster).
  constexpr bool HOLD = !CACHED && 8 * (T1 * T1 + (R1 == R2 ? 0 : T2 * T2)) <= 40;
  FragSet<R1, CACHED, HOLD> F1;
  FragSet<R2, CACHED, HOLD && R1 != R2> F2;
  F1.init(ftab, lane);
  F2.init(ftab, lane);
  auto f1 = [&](int a, int b, int k) { return F1.get(ftab, a, b, k, lane); };
  auto f2 = [&](int a, int b, int k) {
    if constexpr (R1 == R2) return F1.get(ftab, a, b, k, lane);
    else return F2.get(ftab, a, b, k, lane);
  };
  // The twiddles after the stage over n1 and after the inverse over k2 do not depend on
  // the row: w^(R0 k1 n2) at (k1, n2) = (16nt + c, 16t + 4g + v) and (16t + 4g + v, 16nt + c),
  // the same values when R1 == R2. With one tile per axis (R1 = R2 = 16) they are
  // evaluated once per wavefront, with their common scale 1/sqrt(16), instead of twice
  // per row.
  constexpr bool SHARED_TW = T1 == 1 && T2 == 1;
  static_assert(!SHARED_TW || sc1 == sc2, "one tile per axis: equal radices");
  float twr[4], twi[4];
  if constexpr (SHARED_TW) twiddle4<N>(R0 * c, 4 * g, sc1, twr, twi);
  auto tw_n1 = [&](int nt, int t2, float sc, float* wr, float* wi) {
    if constexpr (SHARED_TW) {
#pragma unroll
      for (int v = 0; v < 4; v++) {
        wr[v] = twr[v];
        wi[v] = twi[v];
      }
    } else {
      twiddle4<N>(R0 * (16 * nt + c), 16 * t2 + 4 * g, sc, wr, wi);
    }
  };
  auto twiddle = [](const f4& er, const f4& ei, const float* wr, const float* wi, float* xr, float* xi) {
#pragma unroll
    for (int v = 0; v < 4; v++) {
      xr[v] = er[v] * wr[v] - ei[v] * wi[v];
      xi[v] = er[v] * wi[v] + ei[v] * wr[v];
    }
  };
  // the twiddled accumulators as an fp16 operand (with its remainder when `split`); in the
  // fp16-accumulation mode the packed fp16 product of the raw accumulators
  auto twiddle_pack = [&](const f4& er, const f4& ei, const float* wr, const float* wi, h8& hi, h8& lo,
                          auto split) {
    if (acc16) {
      h4 a, b;
      cmul_hp(er, ei, hw_of(wr, wi), a, b);
      hi = join_h8(a, b);
    } else {
      float xr[4], xi[4];
      twiddle(er, ei, wr, wi, xr, xi);
      pack_operand<decltype(split)::value>(xr, xi, hi, lo);
    }
  };
  // the last twiddle of a row tile, stored as fp16 into the row's block at pos
  auto twiddle_store = [&](const f4& zr, const f4& zi, const float* wr, const float* wi, int pos) {
    h4 hr, hi;
    if (acc16) {
      cmul_hp(zr, zi, hw_of(wr, wi), hr, hi);
    } else {
      float xr[4], xi[4];
      twiddle(zr, zi, wr, wi, xr, xi);
      hr = to_h4(xr);
      hi = to_h4(xi);
    }
    *reinterpret_cast<h4*>(re + pos) = hr;
    *reinterpret_cast<h4*>(im + pos) = hi;
  };
  using SBT = std::integral_constant<bool, SB != 0>;
  using SET = std::integral_constant<bool, SE != 0>;
  // A row's spectrum (kernel order, 2 KB per tile) is read from L2 while the row
  // before it is computed: with one tile per axis the loads are issued one row ahead
  // (double-buffered); otherwise at the start of their own row, in flight while the
  // stage over n1 runs.
  constexpr int KQB = T1 * T2 == 1 && ROWS > 1 ? 2 : 1;
  // rows per step (RP below): plans with one 16x16 tile per row only; with more tiles per
  // row, two rows at a time took more VGPRs than the occupancy allows (L = 8192: 13-15%
  // slower) or gained nothing (L = 16384: 2% slower)
  constexpr int RPK = T1 * T2 != 1              ? 1
                      : ROWS % SFFFT_WG_ROWS == 0 ? SFFFT_WG_ROWS
                      : ROWS % 2 == 0             ? 2
                                                  : 1;
  float4 kq[RPK > 1 ? RPK : KQB][T1][T2][2];
  auto load_row_spectrum = [&](int k0, float4 (*q)[T2][2]) {
#pragma unroll
    for (int t1 = 0; t1 < T1; t1++)
#pragma unroll
      for (int mt = 0; mt < T2; mt++) load_k4(K + (size_t)((k0 * T1 + t1) * T2 + mt) * 256, lane, q[t1][mt]);
  };
  if constexpr (KQB == 2 && RPK == 1) load_row_spectrum(wave * ROWS, kq[0]);
  // The last twiddles of consecutive rows, w^(k0 m) and w^((k0 + 1) m), differ by the
  // factor w^m: with one tile per axis the wavefront evaluates the first row's and the
  // factors once, and steps from row to row with one complex product per value. It holds
  // 16 more VGPRs through the rows: measured faster with 8 rows per wavefront (64x16x16),
  // slower with 4 (32x16x16, where it costs a workgroup per CU).
  constexpr bool REC = T1 * T2 == 1 && ROWS >= 8;
  float lr[4], li[4], fr[4], fi[4];
  if constexpr (REC) {
    const int m0 = 4 * g * R2 + c;  // lane value v: m = m0 + v R2
    twiddle4e<N>(wave * ROWS * m0, wave * ROWS * R2, sc1, lr, li);
    twiddle4e<N>(m0, R2, 1.f, fr, fi);
  }
  // Two forms of the same row loop. One row per step keeps the loop that the multi-tile
  // plans were tuned with: the several-row form, even with one row per step, changes how
  // the compiler schedules and allocates them (up to 5 more spills in some variants).
  if constexpr (RPK == 1) {
#pragma unroll
    for (int i = 0; i < ROWS; i++) {
      const int k0 = wave * ROWS + i;  // each wavefront owns ROWS consecutive rows
      const int rb = k0 * P::ROW;
      if constexpr (KQB == 2) {
        if (i + 1 < ROWS) load_row_spectrum(k0 + 1, kq[(i + 1) & 1]);
      } else {
        load_row_spectrum(k0, kq[0]);
      }
      // stage over n1: A[n2][n1] from the row's [n2 ^ (k0 & 15)][n1] block
      h8 b[T1][T2][1 + SB];  // [k1 tile][n2 tile][hi, lo]: B operands of the stage over n2
      {
        h8 a[T2][T1];
#pragma unroll
        for (int t2 = 0; t2 < T2; t2++)
#pragma unroll
          for (int ks = 0; ks < T1; ks++)
            a[t2][ks] = lds_frag(re, im, rb + (16 * t2 + (c ^ (k0 & 15))) * P::PA + 16 * ks + 4 * g);
#pragma unroll
        for (int t2 = 0; t2 < T2; t2++) {
#pragma unroll
          for (int nt = 0; nt < T1; nt++) {
            f4 dr = {0.f, 0.f, 0.f, 0.f}, di = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < T1; ks++) {
              dr = mfma(a[t2][ks], f1(nt, ks, 0), dr);
              di = mfma(a[t2][ks], f1(nt, ks, 1), di);
            }
            float wr[4], wi[4];
            tw_n1(nt, t2, sc1, wr, wi);
            twiddle_pack(dr, di, wr, wi, b[nt][t2][0], b[nt][t2][SB], SBT{});
          }
        }
      }
      // stage over n2, spectrum, inverse over k2
      h8 e[T2][T1][1 + SE];  // [n2 tile][k1 tile][hi, lo]: B operands of the inverse over k1
#pragma unroll
      for (int t1 = 0; t1 < T1; t1++) {
        f4 dr[T2], di[T2];
#pragma unroll
        for (int mt = 0; mt < T2; mt++) {
          dr[mt] = (f4){0.f, 0.f, 0.f, 0.f};
          di[mt] = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < T2; ks++)
#pragma unroll
            for (int p = 0; p <= SB; p++) {
              dr[mt] = mfma(f2(mt, ks, 0), b[t1][ks][p], dr[mt]);
              di[mt] = mfma(f2(mt, ks, 1), b[t1][ks][p], di[mt]);
            }
        }
        h8 a2[T2], a2lo[SA ? T2 : 1];
        spectrum_product<T2, SA>(dr, di, kq[KQB == 2 ? i & 1 : 0][t1], a2, a2lo, acc16);
#pragma unroll
        for (int nt = 0; nt < T2; nt++) {
          f4 er = {0.f, 0.f, 0.f, 0.f}, ei = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int mt = 0; mt < T2; mt++) {
            er = mfma(a2[mt], f2(nt, mt, 0), er);
            ei = mfma(a2[mt], f2(nt, mt, 1), ei);
            if constexpr (SA) {
              er = mfma(a2lo[mt], f2(nt, mt, 0), er);
              ei = mfma(a2lo[mt], f2(nt, mt, 1), ei);
            }
          }
          float wr[4], wi[4];
          tw_n1(nt, t1, sc2, wr, wi);
          twiddle_pack(er, ei, wr, wi, e[nt][t1][0], e[nt][t1][SE], SET{});
        }
      }
      // inverse over k1 and the last twiddle
      debug_lds_fence();  // the row's reads (stage over n1) before its write-back below
#pragma unroll
      for (int nt = 0; nt < T2; nt++) {
#pragma unroll
        for (int mt = 0; mt < T1; mt++) {
          f4 zr = {0.f, 0.f, 0.f, 0.f}, zi = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < T1; ks++)
#pragma unroll
            for (int p = 0; p <= SE; p++) {
              zr = mfma(f1(mt, ks, 0), e[nt][ks][p], zr);
              zi = mfma(f1(mt, ks, 1), e[nt][ks][p], zi);
            }
          // lane value v is n1 = 16mt + 4g + v, n2 = 16nt + c: m = n1 R2 + n2
          float wr[4], wi[4];
          if constexpr (REC) {
#pragma unroll
            for (int v = 0; v < 4; v++) wr[v] = lr[v], wi[v] = li[v];
            if (i + 1 < ROWS) cmul4(lr, li, fr, fi);
          } else {
            twiddle4e<N>(k0 * ((16 * mt + 4 * g) * R2 + 16 * nt + c), k0 * R2, sc1, wr, wi);
          }
          // back into the row's own block, [n2][n1]: only this wavefront reads the row,
          // and all of its input is in registers by now
          twiddle_store(zr, zi, wr, wi, rb + (16 * nt + c) * P::PA + 16 * mt + 4 * g);
        }
      }
    }
  } else {
    // Rows are taken RP at a time: the operand reads of all of a step's rows come before any
    // of their write-backs, so the compiler can interleave the rows' independent chains (one
    // row's write-back to LDS would otherwise order it before the next row's reads, as it
    // cannot tell the rows' swizzled addresses apart). Each row's arithmetic is the same for
    // any RP, and the last twiddles step from row to row in the same order.
    constexpr int RP = RPK;
#pragma unroll
    for (int i0 = 0; i0 < ROWS; i0 += RP) {
      int k0[RP], rb[RP];
#pragma unroll
      for (int u = 0; u < RP; u++) {
        k0[u] = wave * ROWS + i0 + u;  // each wavefront owns ROWS consecutive rows
        rb[u] = k0[u] * P::ROW;
      }
#pragma unroll
      for (int u = 0; u < RP; u++) load_row_spectrum(k0[u], kq[u]);  // the step's rows' spectra
      // stage over n1: A[n2][n1] from the row's [n2 ^ (k0 & 15)][n1] block
      h8 b[RP][T1][T2][1 + SB];  // [row][k1 tile][n2 tile][hi, lo]: B operands of the stage over n2
      {
        h8 a[RP][T2][T1];
#pragma unroll
        for (int u = 0; u < RP; u++)
#pragma unroll
          for (int t2 = 0; t2 < T2; t2++)
#pragma unroll
            for (int ks = 0; ks < T1; ks++)
              a[u][t2][ks] = lds_frag(re, im, rb[u] + (16 * t2 + (c ^ (k0[u] & 15))) * P::PA + 16 * ks + 4 * g);
#pragma unroll
        for (int t2 = 0; t2 < T2; t2++) {
#pragma unroll
          for (int nt = 0; nt < T1; nt++) {
#pragma unroll
            for (int u = 0; u < RP; u++) {
              f4 dr = {0.f, 0.f, 0.f, 0.f}, di = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
              for (int ks = 0; ks < T1; ks++) {
                dr = mfma(a[u][t2][ks], f1(nt, ks, 0), dr);
                di = mfma(a[u][t2][ks], f1(nt, ks, 1), di);
              }
              float wr[4], wi[4];
              tw_n1(nt, t2, sc1, wr, wi);
              twiddle_pack(dr, di, wr, wi, b[u][nt][t2][0], b[u][nt][t2][SB], SBT{});
            }
          }
        }
      }
      // stage over n2, spectrum, inverse over k2
      h8 e[RP][T2][T1][1 + SE];  // [row][n2 tile][k1 tile][hi, lo]: B operands of the inverse over k1
#pragma unroll
      for (int t1 = 0; t1 < T1; t1++) {
#pragma unroll
        for (int u = 0; u < RP; u++) {
          f4 dr[T2], di[T2];
#pragma unroll
          for (int mt = 0; mt < T2; mt++) {
            dr[mt] = (f4){0.f, 0.f, 0.f, 0.f};
            di[mt] = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < T2; ks++)
#pragma unroll
              for (int p = 0; p <= SB; p++) {
                dr[mt] = mfma(f2(mt, ks, 0), b[u][t1][ks][p], dr[mt]);
                di[mt] = mfma(f2(mt, ks, 1), b[u][t1][ks][p], di[mt]);
              }
          }
          h8 a2[T2], a2lo[SA ? T2 : 1];
          spectrum_product<T2, SA>(dr, di, kq[u][t1], a2, a2lo, acc16);
#pragma unroll
          for (int nt = 0; nt < T2; nt++) {
            f4 er = {0.f, 0.f, 0.f, 0.f}, ei = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int mt = 0; mt < T2; mt++) {
              er = mfma(a2[mt], f2(nt, mt, 0), er);
              ei = mfma(a2[mt], f2(nt, mt, 1), ei);
              if constexpr (SA) {
                er = mfma(a2lo[mt], f2(nt, mt, 0), er);
                ei = mfma(a2lo[mt], f2(nt, mt, 1), ei);
              }
            }
            float wr[4], wi[4];
            tw_n1(nt, t1, sc2, wr, wi);
            twiddle_pack(er, ei, wr, wi, e[u][nt][t1][0], e[u][nt][t1][SE], SET{});
          }
        }
      }
      // inverse over k1 and the last twiddle
      debug_lds_fence();  // the rows' reads (stage over n1) before their write-back below
#pragma unroll
      for (int u = 0; u < RP; u++) {
#pragma unroll
        for (int nt = 0; nt < T2; nt++) {
#pragma unroll
          for (int mt = 0; mt < T1; mt++) {
            f4 zr = {0.f, 0.f, 0.f, 0.f}, zi = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < T1; ks++)
#pragma unroll
              for (int p = 0; p <= SE; p++) {
                zr = mfma(f1(mt, ks, 0), e[u][nt][ks][p], zr);
                zi = mfma(f1(mt, ks, 1), e[u][nt][ks][p], zi);
              }
            // lane value v is n1 = 16mt + 4g + v, n2 = 16nt + c: m = n1 R2 + n2
            float wr[4], wi[4];
            if constexpr (REC) {
#pragma unroll
              for (int v = 0; v < 4; v++) wr[v] = lr[v], wi[v] = li[v];
              if (i0 + u + 1 < ROWS) cmul4(lr, li, fr, fi);
            } else {
              twiddle4e<N>(k0[u] * ((16 * mt + 4 * g) * R2 + 16 * nt + c), k0[u] * R2, sc1, wr, wi);
            }
            // back into the row's own block, [n2][n1]: only this wavefront reads the row,
            // and all of its input is in registers by now
            twiddle_store(zr, zi, wr, wi, rb[u] + (16 * nt + c) * P::PA + 16 * mt + 4 * g);
          }
        }
      }
    }
  }
}

// ---- Phase 3: last inverse stage over k0, first L outputs only -----------------
// (src/sffft.cu:144,165,180-181,279). Reads conj(W)[m][k0]; y = Re of the inverse
// (the second sequence of a pair is the imaginary part).
template <class P, int NW, int NSEQ, class TIO, bool CACHED>
__device__ __forceinline__ void phase3(TIO* __restrict__ ya, TIO* __restrict__ yb, const _Float16* re,
                                       const _Float16* im, const h8* __restrict__ ftab, int acc16, int lane,
                                       int wave) {
  constexpr int R0 = P::R0, M = P::M, MT = M / 16, NT = R0 >= 32 ? R0 / 32 : 1, KS = R0 / 16;
  constexpr float sc0 = R0 == 16 ? 0.25f : R0 == 32 ? 0.17677669529663687f : 0.125f;
  const int r = lane & 15, g = lane >> 4;
  auto tile = [&](const h8* a, int mt, int nt) {
    f4 zr = {0.f, 0.f, 0.f, 0.f}, zi = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
      zr = mfma(a[ks], cf_frag<R0, CACHED>(ftab, nt, ks, 0, lane), zr);
      if constexpr (NSEQ == 2) zi = mfma(a[ks], cf_frag<R0, CACHED>(ftab, nt, ks, 1, lane), zi);
    }
    zr = round_acc(zr, acc16);
    if constexpr (NSEQ == 2) zi = round_acc(zi, acc16);
    const int n0 = 16 * nt + r;
    if (n0 < R0 / 2) {
      const int o = n0 * M + 16 * mt + 4 * g;
      // Plain (write-back) stores: the 64- or 32-byte pieces of one output line come
      // from different wavefronts, and L2 merges them before they reach HBM
      // (streaming stores would write each piece separately).
      if constexpr (sizeof(TIO) == 4) {
        *reinterpret_cast<f4*>(ya + o) = zr * sc0;
        if constexpr (NSEQ == 2) *reinterpret_cast<f4*>(yb + o) = zi * -sc0;
      } else {
        *reinterpret_cast<u32x2*>(ya + o) = f4_to_bf16x4(zr * sc0);
        if constexpr (NSEQ == 2) *reinterpret_cast<u32x2*>(yb + o) = f4_to_bf16x4(zi * -sc0);
      }
    }
  };
  auto load = [&](int mt, h8* a) {
    if constexpr (P::S == 3) {
      // A[m][k0] from the rows [k0][n2][n1] that phase 2 wrote: four k0 per lane, one
      // row apart, read as 16-bit elements
      constexpr int R2 = P::R2;
      const int m = 16 * mt + r, base = (m % R2) * P::PA + m / R2;
#pragma unroll
      for (int ks = 0; ks < KS; ks++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int at = (16 * ks + 4 * g + j) * P::ROW + base;
          a[ks][j] = re[at];
          a[ks][4 + j] = im[at];
        }
    } else {
#pragma unroll
      for (int ks = 0; ks < KS; ks++) a[ks] = lds_frag(re, im, (16 * mt + r) * P::PB + 16 * ks + 4 * g);
    }
  };
  if constexpr (MT >= NW) {
    for (int mt = wave; mt < MT; mt += NW) {
      h8 a[KS];
      load(mt, a);
#pragma unroll
      for (int nt = 0; nt < NT; nt++) tile(a, mt, nt);
    }
  } else {
    for (int u = wave; u < MT * NT; u += NW) {
      const int mt = u / NT, nt = u % NT;
      h8 a[KS];
      load(mt, a);
      tile(a, mt, nt);
    }
  }
}

// ---- The fused kernel (src/sffft.cu:243-280) ------------------------------------
// Block -> (channel h, batch pair bp). The reference orders blocks batch-fastest
// (src/sffft.cu:249) so one channel's spectrum is reused from cache. Workgroups are
// dispatched to the 8 XCDs round-robin (block i -> XCD i mod 8), each XCD with its
// own L2, so when H is a multiple of 8 the B/NSEQ workgroups of a channel are given
// consecutive slots of one XCD: the spectrum of that channel is fetched into one L2.
__device__ __forceinline__ void block_to_item(int i, int H, int BP, int& h, int& bp) {
  if ((H & 7) == 0) {
    const int x = i & 7, j = i >> 3, q = j / BP;
    h = 8 * q + x;
    bp = j - q * BP;
  } else {
    h = i / BP;
    bp = i - h * BP;
  }
}

// Wavefronts per SIMD that the workgroup's LDS allows on one CU (160 KB), at most 8.
template <class P, int NW>
__host__ __device__ constexpr int lds_waves_per_simd() {
  return (163840 / P::LDS_BYTES) * NW / 4 < 1 ? 1 : (163840 / P::LDS_BYTES) * NW / 4 > 8 ? 8 : (163840 / P::LDS_BYTES) * NW / 4;
}

// fp32 splits of a three-stage plan with fp32 I/O (bits as SFFFT_FP32_SPLITS). At N = 8192
// (L = 4096) the pair plans measured 4.7e-4 (0.94 of the fp32 bound) with the input split
// alone; the operand of the inverse stage over k1 also carrying its remainder (bit 2,
// twice that stage's MFMAs) brings them to 4.4e-4 for 5-8% time. The other lengths stay
// at or below 4.3e-4 without it.
template <class P>
constexpr int fp32_splits() {
  return SFFFT_FP32_SPLITS | (P::S == 3 && P::N == 8192 ? 4 : 0);
}

// grid = H * (B / NSEQ) workgroups of 64*NW lanes; one sequence (NSEQ = 1) or one
// pair of sequences of the same channel (NSEQ = 2) per workgroup.
// ACC16 (fp16-accumulation mode) is a compile-time choice: as a runtime flag every
// accumulator rounding was a branch, and the branches cut each phase into one
// scheduling block per tile. WPE is the wavefronts per SIMD the register allocation
// must allow (the LDS-limited occupancy, or 1 for no limit): without it the schedule
// of the longer blocks can take more VGPRs than that occupancy leaves.
template <class P, int NW, int NSEQ, class TIO, bool CACHED, bool ACC16, int WPE>
__global__ void __launch_bounds__(64 * NW, WPE)
    fftconv_kernel(const TIO* __restrict__ u, const float2* __restrict__ kf, TIO* __restrict__ y, int B, int H,
                   const h8* __restrict__ ftab) {
  constexpr int acc16 = ACC16 ? 1 : 0;
  __shared__ __attribute__((aligned(16))) _Float16 lds[2 * P::PLANE];
  _Float16* re = lds;
  _Float16* im = lds + P::PLANE;
  // the wavefront index is uniform: a scalar register, so the work split derived from
  // it runs on the scalar unit
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int h, bp;
  block_to_item(blockIdx.x, H, B / NSEQ, h, bp);
  const size_t row_a = ((size_t)(bp * NSEQ) * H + h) * P::L;
  const size_t row_b = NSEQ == 2 ? row_a + (size_t)H * P::L : row_a;
  const float2* K = kf + (size_t)h * P::N;
  // fp32 input as fp16 value plus remainder (fp32 accumulation; the fp16-accumulation mode
  // keeps its one rounding)
  constexpr bool SPLIT_IN = sizeof(TIO) == 4 && !ACC16 && (SFFFT_FP32_SPLITS & 8);
  // every global load of the input (and, for two-stage plans, of the spectrum) is
  // issued before any computation, so their latencies overlap
  P1Frags<P, NW, NSEQ, CACHED> fr;
  fr.load(ftab, lane, wave);
  P1Data<P, NW, NSEQ, TIO> ad;
  p1_prefetch<P, NW, NSEQ, TIO>(u + row_a, u + row_b, ad, lane, wave);
  if constexpr (P::S == 2) {
    KData2<P, NW> kd;
    k_prefetch_s2<P, NW>(K, kd, lane, wave);
    phase1<P, NW, NSEQ, TIO, CACHED, SPLIT_IN>(ad, fr, re, im, ftab, acc16, lane, wave);
    __syncthreads();
    phase2_s2<P, NW, CACHED, sizeof(TIO) == 4 && !ACC16>(re, im, kd, ftab, acc16, lane, wave);
  } else {
    phase1<P, NW, NSEQ, TIO, CACHED, SPLIT_IN>(ad, fr, re, im, ftab, acc16, lane, wave);
    __syncthreads();
    phase2_s3<P, NW, CACHED, sizeof(TIO) == 4 && !ACC16 ? fp32_splits<P>() : 0>(re, im, K, ftab, acc16, lane, wave);
  }
  __syncthreads();
  phase3<P, NW, NSEQ, TIO, CACHED>(y + row_a, y + row_b, re, im, ftab, acc16, lane, wave);
}

// Kernel-order spectrum index -> digits (k0, k1, k2) of the frequency
// k = k0 + R0*k1 + R0*R1*k2 (the digit order of src/sffft.cu:283-288, laid out
// in the register order in which the fused kernel consumes it).
template <class P>
__host__ __device__ inline void kernel_order_digits(int idx, int& k0, int& k1, int& k2) {
  const int v = idx & 3, lane = (idx >> 2) & 63, rest = idx >> 8;
  const int c = lane & 15, g = lane >> 4;
  if constexpr (P::S == 2) {
    const int T1 = P::R1 / 16, mt = rest % T1, s = rest / T1;
    k0 = 16 * s + c;
    k1 = 16 * mt + 4 * g + v;
    k2 = 0;
  } else {
    const int T1 = P::R1 / 16, T2 = P::R2 / 16;
    const int mt = rest % T2, t1 = (rest / T2) % T1;
    k0 = rest / (T2 * T1);
    k1 = 16 * t1 + c;
    k2 = 16 * mt + 4 * g + v;
  }
}

}  // namespace sffft
