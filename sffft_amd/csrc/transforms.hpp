// Standalone complex transforms and the 2-D circular convolution built on them.
//
// The reference lists standalone forward/inverse FFTs and 2-D convolution as not
// exposed (README.md:174); these have no counterpart there. They favour accuracy over
// speed: each stage is a radix-R DFT along one digit of the position, evaluated in fp64
// (an in-register radix-2 FFT of the R points per thread, fp64 twiddles) and stored as
// complex64 between stages (relative error ~1e-7). The fused convolution kernels, with
// fp16 MFMA operands, are separate.
//
// Algorithm: N = r[0] * r[1] * ... * r[S-1] (powers of two, 16s first). Decimation in
// frequency: stage J transforms digit J (stride s_J = r[J+1] * ... * r[S-1]) and, before
// the next stage, multiplies by w_{r[J] s_J}^(k_J * (p mod s_J)). After the last stage
// position p = sum_J k_J s_J holds frequency k = k_0 + r[0] (k_1 + r[1] (k_2 + ...)), so
// the last stage writes each value to its natural-order slot directly. Contiguous sequences
// of up to ONEPASS_MAX_N points run every stage in LDS in one launch (line_kernel); longer
// or strided ones take one launch per stage (stage_kernel), through a workspace.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sffft {
namespace xf {

#ifndef SFFFT_XF_MAX_RADIX
#define SFFFT_XF_MAX_RADIX 16
#endif
constexpr int MAX_RADIX = SFFFT_XF_MAX_RADIX;
constexpr int MAX_STAGES = 6;
constexpr long long MAX_N = 1LL << 24;
constexpr long long MAX_ELEMS = 1LL << 31;  // sequences * N per call

constexpr bool stages_cover_max_n() {
  long long n = 1;
  for (int i = 0; i < MAX_STAGES; i++) n *= MAX_RADIX;
  return n >= MAX_N;
}
static_assert(stages_cover_max_n(), "MAX_STAGES stages of MAX_RADIX must reach MAX_N");

struct Radices {
  int S;
  int r[MAX_STAGES];
};

// N a power of two in [2, 2^24]: radix-MAX_RADIX stages, then the remainder.
inline bool split(long long N, Radices* out) {
  if (N < 2 || N > MAX_N || (N & (N - 1))) return false;
  Radices d{0, {1, 1, 1, 1, 1, 1}};
  long long rest = N;
  while (rest > MAX_RADIX) {
    if (d.S == MAX_STAGES - 1) return false;  // never write past r[MAX_STAGES - 1]
    d.r[d.S++] = MAX_RADIX;
    rest /= MAX_RADIX;
  }
  d.r[d.S++] = (int)rest;
  *out = d;
  return true;
}

// Element n of sequence s sits at (s / inner) * dist_outer + (s % inner) * dist_inner +
// n * stride (complex elements). seq_fast: consecutive threads take consecutive
// sequences (set when sequences interleave more tightly than their elements, as the
// columns of a row-major matrix do), and the stage workspace is then laid out [p][s]
// so that every stage reads and writes consecutive addresses across a wavefront.
struct Seqs {
  long long nseq, inner, dist_inner, dist_outer, stride;
  int seq_fast;
  __host__ __device__ long long base(long long s) const {
    return (s / inner) * dist_outer + (s % inner) * dist_inner;
  }
};

// The radix-R DFT of one line's R points, in registers, shared by both kernels below:
// radix-2 decimation in frequency over log2(R) levels, natural input order, bit-reversed
// output order, in fp64 with w_m^j = w_T^(j * T / m) read from a table of the T-th roots
// of unity. About R*log2(R)/2 complex products instead of the R*R of the dense sum.
// Contraction is off and the complex products are written with fma, so every kernel
// that inlines this rounds in the same places and gets the same bits.
template <int R, int T>
__device__ __forceinline__ void line_dft(double (&vr)[R], double (&vi)[R], const double* wc, const double* ws) {
#pragma clang fp contract(off)
#pragma unroll
  for (int m = R; m >= 2; m >>= 1) {
    const int h = m >> 1, step = T / m;
#pragma unroll
    for (int b = 0; b < R; b += m)
#pragma unroll
      for (int j = 0; j < h; j++) {
        const int i0 = b + j, i1 = i0 + h;
        const double ar = vr[i0], ai = vi[i0], dr = ar - vr[i1], di = ai - vi[i1];
        vr[i0] = ar + vr[i1];
        vi[i0] = ai + vi[i1];
        if (j == 0) {
          vr[i1] = dr;
          vi[i1] = di;
        } else {
          const double c = wc[j * step], sn = ws[j * step];
          vr[i1] = fma(dr, c, -(di * sn));
          vi[i1] = fma(dr, sn, di * c);
        }
      }
  }
}

template <int R>
__device__ __forceinline__ int bitrev(int k) {
  int r = 0;
#pragma unroll
  for (int b = 1; b < R; b <<= 1) r = (r << 1) | ((k & b) ? 1 : 0);
  return r;
}

// Frequency digit k of a non-last stage's line times w_Nj^(k * inner), rounded to
// complex64 once; store(k, value) for k = 0 .. R-1. The twiddles are powers of
// w_Nj^inner = w1c + i w1s, built by recurrence in fp64 (same rounding rule as line_dft).
template <int R, class Store>
__device__ __forceinline__ void twiddled_outputs_w(const double (&vr)[R], const double (&vi)[R], double w1c,
                                                   double w1s, Store store) {
#pragma clang fp contract(off)
  double wr = 1.0, wi = 0.0;
#pragma unroll
  for (int k = 0; k < R; k++) {
    const int r = bitrev<R>(k);
    store(k, make_float2((float)fma(vr[r], wr, -(vi[r] * wi)), (float)fma(vr[r], wi, vi[r] * wr)));
    const double nr = fma(wr, w1c, -(wi * w1s));
    wi = fma(wr, w1s, wi * w1c);
    wr = nr;
  }
}

// The same with w_Nj^inner evaluated here (one fp64 sincospi of the exact angle).
template <int R, class Store>
__device__ __forceinline__ void twiddled_outputs(const double (&vr)[R], const double (&vi)[R], int inner, int Nj,
                                                 int sign, Store store) {
  double w1s, w1c;
  sincospi(2.0 * (double)inner / (double)Nj, &w1s, &w1c);
  twiddled_outputs_w<R>(vr, vi, w1c, sign * w1s, store);
}

template <int R>
__global__ void __launch_bounds__(128)
    stage_kernel(const float2* in, float2* out, float2* work, Seqs q, Radices d, int J, int N, int sign,
                 float scale) {
  __shared__ double wc[R], ws[R];
  for (int i = threadIdx.x; i < R; i += blockDim.x) {
    double sn, c;
    sincospi(2.0 * (double)i / (double)R, &sn, &c);
    wc[i] = c;
    ws[i] = sign * sn;  // w_R^i = c + i * ws[i]
  }
  __syncthreads();
  const int S = d.S;
  int sJ = 1;
  for (int i = J + 1; i < S; i++) sJ *= d.r[i];
  const int lines = N / R;
  const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= q.nseq * lines) return;
  const long long s = q.seq_fast ? gid % q.nseq : gid / lines;
  const int l = (int)(q.seq_fast ? gid / q.nseq : gid % lines);
  const int inner = l % sJ, outer = l / sJ;
  const int base = outer * R * sJ + inner;
  auto widx = [&](int p) -> long long { return q.seq_fast ? (long long)p * q.nseq + s : s * N + p; };
  float2 x[R];
  if (J == 0) {
    const float2* src = in + q.base(s);
#pragma unroll
    for (int t = 0; t < R; t++) x[t] = src[(long long)(base + t * sJ) * q.stride];
  } else {
#pragma unroll
    for (int t = 0; t < R; t++) x[t] = work[widx(base + t * sJ)];
  }
  const bool last = J == S - 1;
  // natural-order frequency of this line's first output (last stage: sJ = 1, inner = 0)
  long long kbase = 0, wlast = 1;
  if (last) {
    int sj = N;
    long long w = 1;
    for (int j = 0; j < S - 1; j++) {
      sj /= d.r[j];
      kbase += (long long)((base / sj) % d.r[j]) * w;
      w *= d.r[j];
    }
    wlast = w;
  }
  float2* dst = out + q.base(s);
  const int Nj = R * sJ;
  double vr[R], vi[R];
#pragma unroll
  for (int t = 0; t < R; t++) {
    vr[t] = (double)x[t].x;
    vi[t] = (double)x[t].y;
  }
  line_dft<R, R>(vr, vi, wc, ws);
  if (last) {
#pragma unroll
    for (int k = 0; k < R; k++) {
      const int r = bitrev<R>(k);
      dst[(kbase + (long long)k * wlast) * q.stride] = make_float2((float)(vr[r] * scale), (float)(vi[r] * scale));
    }
  } else {
    // twiddle w_Nj^(k * inner) before the next stage
    twiddled_outputs<R>(vr, vi, inner, Nj, sign, [&](int k, float2 v) { work[widx(base + k * sJ)] = v; });
  }
}

// ---- one pass over short contiguous lines ------------------------------------------
// Sequences of N <= ONEPASS_MAX_N elements at unit stride are transformed in one launch: a
// workgroup loads G = max(1, ONEPASS_SLOTS / N) whole sequences into LDS, runs every stage
// there and writes the natural-order result back, so each sequence crosses HBM once
// each way instead of once per stage. The stages are those of stage_kernel (the same
// radix split, fp64 line DFTs, twiddle recurrences and complex64 rounding between
// stages), so the results are bit-identical to the staged path. One LDS slot of padding
// per 16 elements keeps the threads of the last stage (R consecutive elements each) on
// different banks.
constexpr int ONEPASS_MAX_N = 16384;  // 136 KB of LDS
constexpr int ONEPASS_SLOTS = 4096;

__device__ __forceinline__ int lpad(int p) { return p + (p >> 4); }

template <int N>
struct LineGeom {
  static constexpr int G = N >= ONEPASS_SLOTS ? 1 : ONEPASS_SLOTS / N;  // sequences per workgroup
  static constexpr int SLOTS = G * N;
  // one thread per radix-16 line: 256 threads, 512 at N = 8192, 1024 at N = 16384
  static constexpr int THREADS = SLOTS / MAX_RADIX;
  static constexpr int LDS = SLOTS + SLOTS / 16;
  // twiddle bases of the non-last stages: w_N^j for j < N / 16 (w_Nj^inner = w_N^(inner N/Nj))
  static constexpr int TW = N / MAX_RADIX > 1 ? N / MAX_RADIX : 1;
  // radix of the stage whose remaining product of radices is REST (16s first)
  static constexpr int radix(int rest) { return rest > MAX_RADIX ? MAX_RADIX : rest; }
};

// One stage over the workgroup's lines: REST is the product of this and the later
// radices (REST = N at the first stage), R this stage's radix, sJ = REST / R its stride.
// tc, ts: the workgroup's table of w_N^j = tc[j] + i sign ts[j], j < N/16. A line's twiddle
// base w_REST^inner is entry inner * N/REST: sincospi of 2j/N there and of 2 inner/REST in
// the staged kernel are the same exact fp64 argument, so both paths get the same bits.
// G sequences of N in buf, THREADS threads (the one-pass kernel's geometry by default).
template <int N, int REST, int G = LineGeom<N>::G, int THREADS = LineGeom<N>::THREADS>
__device__ __forceinline__ void line_stage(float2* buf, const double* wc, const double* ws, const double* tc,
                                           const double* ts, int sign, float scale) {
  constexpr int R = LineGeom<N>::radix(REST), sJ = REST / R, LPS = N / R;
  constexpr int LINES = G * LPS;
  constexpr bool LAST = REST == R;
  for (int li = threadIdx.x; li < LINES; li += THREADS) {
    const int g = li / LPS, l = li - g * LPS;
    const int inner = l % sJ, base = g * N + (l / sJ) * REST + inner;
    double vr[R], vi[R];
#pragma unroll
    for (int t = 0; t < R; t++) {
      const float2 x = buf[lpad(base + t * sJ)];
      vr[t] = (double)x.x;
      vi[t] = (double)x.y;
    }
    line_dft<R, MAX_RADIX>(vr, vi, wc, ws);
    if constexpr (LAST) {
      // in place, scaled: element base + k holds frequency digit k of this line
#pragma unroll
      for (int k = 0; k < R; k++) {
        const int r = bitrev<R>(k);
        buf[lpad(base + k)] = make_float2((float)(vr[r] * scale), (float)(vi[r] * scale));
      }
    } else {
      const int j = inner * (N / REST);
      twiddled_outputs_w<R>(vr, vi, tc[j], sign * ts[j], [&](int k, float2 v) { buf[lpad(base + k * sJ)] = v; });
    }
  }
  __syncthreads();
  if constexpr (!LAST) line_stage<N, REST / R, G, THREADS>(buf, wc, ws, tc, ts, sign, scale);
}

// Position in the line, after the last stage, of natural-order frequency f: the digits
// of f below the last stage's (f mod W, W the product of all radices but the last) name
// the line, reversed into its base position; the last digit is the element within it.
template <int N>
__device__ __forceinline__ int line_position(int f) {
  int W = 1, rest = N;
  while (rest > MAX_RADIX) {
    W *= MAX_RADIX;
    rest /= MAX_RADIX;
  }
  int kb = f % W, base = 0, sj = N;
  for (int w = 1; w < W; w *= MAX_RADIX) {
    sj /= MAX_RADIX;
    base += ((kb / w) % MAX_RADIX) * sj;
  }
  return base + f / W;
}

template <int N>
__global__ void __launch_bounds__(LineGeom<N>::THREADS)
    line_kernel(const float2* in, float2* out, Seqs q, int sign, float scale) {
  typedef LineGeom<N> LG;
  __shared__ float2 buf[LG::LDS];
  __shared__ double wc[MAX_RADIX], ws[MAX_RADIX];
  __shared__ double tc[LG::TW], ts[LG::TW];
  if (threadIdx.x < MAX_RADIX) {
    double sn, c;
    sincospi(2.0 * (double)threadIdx.x / (double)MAX_RADIX, &sn, &c);
    wc[threadIdx.x] = c;
    ws[threadIdx.x] = sign * sn;
  }
  // one sincospi per table entry instead of one per line and stage
  for (int j = threadIdx.x; j < LG::TW; j += LG::THREADS) {
    double sn, c;
    sincospi(2.0 * (double)j / (double)N, &sn, &c);
    tc[j] = c;
    ts[j] = sn;
  }
  const long long s0 = (long long)blockIdx.x * LG::G;
  const int G = q.nseq - s0 < LG::G ? (int)(q.nseq - s0) : LG::G;
  for (int i = threadIdx.x; i < LG::SLOTS; i += LG::THREADS) {
    const int g = i / N;
    buf[lpad(i)] = g < G ? in[q.base(s0 + g) + (i - g * N)] : make_float2(0.f, 0.f);
  }
  __syncthreads();
  line_stage<N, N>(buf, wc, ws, tc, ts, sign, scale);
  for (int i = threadIdx.x; i < G * N; i += LG::THREADS) {
    const int g = i / N, f = i - g * N;
    out[q.base(s0 + g) + f] = buf[lpad(g * N + line_position<N>(f))];
  }
}

template <int N>
inline void launch_line(const float2* in, float2* out, const Seqs& q, int sign, float scale, hipStream_t st) {
  const unsigned grid = (unsigned)((q.nseq + LineGeom<N>::G - 1) / LineGeom<N>::G);
  hipLaunchKernelGGL(line_kernel<N>, dim3(grid), dim3(LineGeom<N>::THREADS), 0, st, in, out, q, sign, scale);
}

inline bool run_lines(const float2* in, float2* out, const Seqs& q, int N, int sign, float scale, hipStream_t st) {
  if (q.stride != 1 || q.seq_fast) return false;
  switch (N) {
    case 2: launch_line<2>(in, out, q, sign, scale, st); return true;
    case 4: launch_line<4>(in, out, q, sign, scale, st); return true;
    case 8: launch_line<8>(in, out, q, sign, scale, st); return true;
    case 16: launch_line<16>(in, out, q, sign, scale, st); return true;
    case 32: launch_line<32>(in, out, q, sign, scale, st); return true;
    case 64: launch_line<64>(in, out, q, sign, scale, st); return true;
    case 128: launch_line<128>(in, out, q, sign, scale, st); return true;
    case 256: launch_line<256>(in, out, q, sign, scale, st); return true;
    case 512: launch_line<512>(in, out, q, sign, scale, st); return true;
    case 1024: launch_line<1024>(in, out, q, sign, scale, st); return true;
    case 2048: launch_line<2048>(in, out, q, sign, scale, st); return true;
    case 4096: launch_line<4096>(in, out, q, sign, scale, st); return true;
    case 8192: launch_line<8192>(in, out, q, sign, scale, st); return true;
    case 16384: launch_line<16384>(in, out, q, sign, scale, st); return true;
    default: return false;
  }
}

// ---- two passes over long contiguous lines ------------------------------------------
// Sequences of ONEPASS_MAX_N < N <= MAX_N points at unit stride: N = N1 * N2 with N1 = 16^k.
// The first k stages move positions only within the N1-point columns p = c + m N2 (c < N2),
// and leave N1 independent blocks of N2 contiguous positions, each of which the remaining
// stages transform as an N2-point sequence (the same twiddles, w_Nj with Nj <= N2). So:
//   pass A (col_kernel): C columns per workgroup, loaded as runs of C points from each of
//   the N1 rows, stages 0..k-1 in LDS with the stage kernel's line DFTs and twiddles (the
//   global inner index c + u N2), written back in place to the workspace;
//   pass B (row_kernel): G blocks per workgroup, the one-pass stages of an N2-point
//   sequence, and block b's frequency f written to k = rev(b) + N1 f, rev reversing b's k
//   base-16 digits; the G blocks have consecutive rev(b), so the writes are runs of G points.
// Each sequence crosses HBM twice each way instead of once per stage, with the staged
// kernels' arithmetic in the same order: the results are bit-identical to them.
constexpr int TWOPASS_MAX_N1 = 4096, TWOPASS_MAX_N2 = 4096;

template <int N1>
struct ColGeom {
  static constexpr int C = N1 >= 1024 ? 4 : 4096 / N1;  // columns per workgroup
  static constexpr int SLOTS = N1 * C;
  static constexpr int THREADS = SLOTS / MAX_RADIX;
};

template <int N2>
struct RowGeom {
  static constexpr int G = N2 >= 1024 ? 4 : 4096 / N2;  // blocks per workgroup
  static constexpr int SLOTS = G * N2;
  static constexpr int THREADS = SLOTS / MAX_RADIX;
  static constexpr int LDS = SLOTS + SLOTS / 16;
};

// stage of pass A whose local stride is LS (N1/16 at the first stage, 1 at the last)
template <int N1, int LS>
__device__ __forceinline__ void col_stage(float2* buf, const double* wc, const double* ws, int c0, int N2,
                                          int sign) {
  constexpr int R = MAX_RADIX, C = ColGeom<N1>::C, LINES = (N1 / R) * C;
  for (int li = threadIdx.x; li < LINES; li += ColGeom<N1>::THREADS) {
    const int j = li % C, l = li / C;  // column j (consecutive across threads), line l of it
    const int lu = l % LS, mb = (l / LS) * R * LS + lu;
    double vr[R], vi[R];
#pragma unroll
    for (int t = 0; t < R; t++) {
      const float2 x = buf[(mb + t * LS) * C + j];
      vr[t] = (double)x.x;
      vi[t] = (double)x.y;
    }
    line_dft<R, R>(vr, vi, wc, ws);
    // the stage kernel's twiddle of this line: inner = p mod sJ, Nj = R sJ, sJ = LS N2
    twiddled_outputs<R>(vr, vi, c0 + j + lu * N2, R * LS * N2, sign,
                        [&](int k, float2 v) { buf[(mb + k * LS) * C + j] = v; });
  }
  __syncthreads();
  if constexpr (LS > 1) col_stage<N1, LS / R>(buf, wc, ws, c0, N2, sign);
}

template <int N1>
__global__ void __launch_bounds__(ColGeom<N1>::THREADS)
    col_kernel(const float2* in, float2* work, Seqs q, int N2, int sign) {
  typedef ColGeom<N1> CG;
  __shared__ float2 buf[CG::SLOTS];
  __shared__ double wc[MAX_RADIX], ws[MAX_RADIX];
  if (threadIdx.x < MAX_RADIX) {
    double sn, c;
    sincospi(2.0 * (double)threadIdx.x / (double)MAX_RADIX, &sn, &c);
    wc[threadIdx.x] = c;
    ws[threadIdx.x] = sign * sn;
  }
  const int per_seq = N2 / CG::C;
  const long long s = blockIdx.x / per_seq;
  const int c0 = (int)(blockIdx.x - s * per_seq) * CG::C;
  const long long N = (long long)N1 * N2;
  const float2* src = in + q.base(s) + c0;
  for (int i = threadIdx.x; i < CG::SLOTS; i += CG::THREADS) {
    const int m = i / CG::C, j = i - m * CG::C;
    buf[i] = src[(long long)m * N2 + j];
  }
  __syncthreads();
  col_stage<N1, N1 / MAX_RADIX>(buf, wc, ws, c0, N2, sign);
  float2* dst = work + s * N + c0;
  for (int i = threadIdx.x; i < CG::SLOTS; i += CG::THREADS) {
    const int m = i / CG::C, j = i - m * CG::C;
    dst[(long long)m * N2 + j] = buf[i];
  }
}

// b's k base-16 digits reversed (an involution)
__device__ __forceinline__ int digit_reverse16(int b, int k) {
  int r = 0;
  for (int i = 0; i < k; i++) {
    r = (r << 4) | (b & 15);
    b >>= 4;
  }
  return r;
}

template <int N2>
__global__ void __launch_bounds__(RowGeom<N2>::THREADS)
    row_kernel(const float2* work, float2* out, Seqs q, int N1, int k, int sign, float scale) {
  typedef RowGeom<N2> RG;
  typedef LineGeom<N2> LG;
  __shared__ float2 buf[RG::LDS];
  __shared__ double wc[MAX_RADIX], ws[MAX_RADIX];
  __shared__ double tc[LG::TW], ts[LG::TW];
  if (threadIdx.x < MAX_RADIX) {
    double sn, c;
    sincospi(2.0 * (double)threadIdx.x / (double)MAX_RADIX, &sn, &c);
    wc[threadIdx.x] = c;
    ws[threadIdx.x] = sign * sn;
  }
  for (int j = threadIdx.x; j < LG::TW; j += RG::THREADS) {
    double sn, c;
    sincospi(2.0 * (double)j / (double)N2, &sn, &c);
    tc[j] = c;
    ts[j] = sn;
  }
  const int per_seq = N1 / RG::G;
  const long long s = blockIdx.x / per_seq;
  const int r0 = (int)(blockIdx.x - s * per_seq) * RG::G;  // rev(b) of the first block
  const long long N = (long long)N1 * N2;
  const float2* src = work + s * N;
  for (int i = threadIdx.x; i < RG::SLOTS; i += RG::THREADS) {
    const int g = i / N2, e = i - g * N2;
    buf[lpad(i)] = src[(long long)digit_reverse16(r0 + g, k) * N2 + e];
  }
  __syncthreads();
  line_stage<N2, N2, RG::G, RG::THREADS>(buf, wc, ws, tc, ts, sign, scale);
  float2* dst = out + q.base(s) + r0;
  for (int i = threadIdx.x; i < RG::SLOTS; i += RG::THREADS) {
    const int f = i / RG::G, g = i - f * RG::G;
    dst[(long long)f * N1 + g] = buf[lpad(g * N2 + line_position<N2>(f))];
  }
}

template <int N1>
inline void launch_cols(const float2* in, float2* work, const Seqs& q, int N2, int sign, hipStream_t st) {
  const unsigned grid = (unsigned)(q.nseq * (N2 / ColGeom<N1>::C));
  hipLaunchKernelGGL(col_kernel<N1>, dim3(grid), dim3(ColGeom<N1>::THREADS), 0, st, in, work, q, N2, sign);
}

template <int N2>
inline void launch_rows(const float2* work, float2* out, const Seqs& q, int N1, int k, int sign, float scale,
                        hipStream_t st) {
  const unsigned grid = (unsigned)(q.nseq * (N1 / RowGeom<N2>::G));
  hipLaunchKernelGGL(row_kernel<N2>, dim3(grid), dim3(RowGeom<N2>::THREADS), 0, st, work, out, q, N1, k, sign,
                     scale);
}

// The column count k (N1 = 16^k) whose passes read and write the longest runs: pass A's
// runs are C points, pass B's G points; both passes within TWOPASS_MAX_N1 / _N2. 0 if none.
inline int two_pass_k(long long N) {
  int best = 0, best_run = 0;
  for (int k = 1; k <= 3; k++) {
    const long long N1 = 1LL << (4 * k), N2 = N / N1;
    if (N1 > TWOPASS_MAX_N1 || N2 > TWOPASS_MAX_N2 || N2 < 16 || N1 * N2 != N) continue;
    const int C = N1 >= 1024 ? 4 : (int)(4096 / N1), G = N2 >= 1024 ? 4 : (int)(4096 / N2);
    if (G > N1 || C > N2) continue;
    const int run = C < G ? C : G;
    if (run > best_run) best = k, best_run = run;
  }
  return best;
}

inline bool run_two_pass(const float2* in, float2* out, float2* work, const Seqs& q, long long N, int sign,
                         float scale, hipStream_t st) {
  if (q.stride != 1 || q.seq_fast || N <= ONEPASS_MAX_N) return false;
  const int k = two_pass_k(N);
  if (!k) return false;
  const int N1 = 1 << (4 * k), N2 = (int)(N / N1);
  switch (N1) {
    case 16: launch_cols<16>(in, work, q, N2, sign, st); break;
    case 256: launch_cols<256>(in, work, q, N2, sign, st); break;
    case 4096: launch_cols<4096>(in, work, q, N2, sign, st); break;
    default: return false;
  }
  switch (N2) {
    case 16: launch_rows<16>(work, out, q, N1, k, sign, scale, st); break;
    case 32: launch_rows<32>(work, out, q, N1, k, sign, scale, st); break;
    case 64: launch_rows<64>(work, out, q, N1, k, sign, scale, st); break;
    case 128: launch_rows<128>(work, out, q, N1, k, sign, scale, st); break;
    case 256: launch_rows<256>(work, out, q, N1, k, sign, scale, st); break;
    case 512: launch_rows<512>(work, out, q, N1, k, sign, scale, st); break;
    case 1024: launch_rows<1024>(work, out, q, N1, k, sign, scale, st); break;
    case 2048: launch_rows<2048>(work, out, q, N1, k, sign, scale, st); break;
    case 4096: launch_rows<4096>(work, out, q, N1, k, sign, scale, st); break;
    default: return false;
  }
  return true;
}

// Workspace of one transform call: the stage results between the first and last stage.
inline long long work_elems(const Seqs& q, long long N) {
  Radices d;
  if (!split(N, &d)) return -1;
  return d.S > 1 ? q.nseq * N : 0;
}

// All stages of one batched 1-D transform; `work` holds work_elems(q, N) complex64.
// `in` may equal `out`: the first stage reads all of `in` before the last one writes.
inline hipError_t run(const float2* in, float2* out, float2* work, const Seqs& q, int N, int inverse, float scale,
                      hipStream_t st) {
  Radices d;
  if (!split(N, &d)) return hipErrorInvalidValue;
  const int sign = inverse ? 1 : -1;
  if (N <= ONEPASS_MAX_N && run_lines(in, out, q, N, sign, scale, st)) return hipGetLastError();
  if (run_two_pass(in, out, work, q, N, sign, scale, st)) return hipGetLastError();
  for (int J = 0; J < d.S; J++) {
    const long long threads = q.nseq * (N / d.r[J]);
    const dim3 grid((unsigned)((threads + 127) / 128)), block(128);
    const float sc = J == d.S - 1 ? scale : 1.f;
    switch (d.r[J]) {
      case 2: hipLaunchKernelGGL(stage_kernel<2>, grid, block, 0, st, in, out, work, q, d, J, N, sign, sc); break;
      case 4: hipLaunchKernelGGL(stage_kernel<4>, grid, block, 0, st, in, out, work, q, d, J, N, sign, sc); break;
      case 8: hipLaunchKernelGGL(stage_kernel<8>, grid, block, 0, st, in, out, work, q, d, J, N, sign, sc); break;
      case 16: hipLaunchKernelGGL(stage_kernel<16>, grid, block, 0, st, in, out, work, q, d, J, N, sign, sc); break;
      case 32: hipLaunchKernelGGL(stage_kernel<32>, grid, block, 0, st, in, out, work, q, d, J, N, sign, sc); break;
      case 64: hipLaunchKernelGGL(stage_kernel<64>, grid, block, 0, st, in, out, work, q, d, J, N, sign, sc); break;
      default: return hipErrorInvalidValue;
    }
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

// Rows then columns of nimg contiguous [N0][N1] arrays; `x` may equal `X`.
inline Seqs rows_of(long long nimg, int N0, int N1) { return Seqs{nimg * N0, nimg * N0, N1, 0, 1, 0}; }
inline Seqs cols_of(long long nimg, int N0, int N1) {
  return Seqs{nimg * N1, N1, 1, (long long)N0 * N1, N1, 1};
}

inline long long work2_elems(long long nimg, int N0, int N1) {
  const long long a = work_elems(rows_of(nimg, N0, N1), N1), b = work_elems(cols_of(nimg, N0, N1), N0);
  if (a < 0 || b < 0) return -1;
  return a > b ? a : b;
}

inline hipError_t run2(const float2* x, float2* X, float2* work, long long nimg, int N0, int N1, int inverse,
                       float scale, hipStream_t st) {
  hipError_t err = run(x, X, work, rows_of(nimg, N0, N1), N1, inverse, 1.f, st);
  if (err != hipSuccess) return err;
  return run(X, X, work, cols_of(nimg, N0, N1), N0, inverse, scale, st);
}

__global__ void widen_kernel(const float* __restrict__ u, float2* __restrict__ w, long long n) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) w[i] = make_float2(u[i], 0.f);
}

// U[b][h][p] *= scale * K[h][p]
__global__ void spectrum_product_kernel(float2* __restrict__ U, const float2* __restrict__ K, long long P, int H,
                                        long long n, float scale) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float2 a = U[i], b = K[((i / P) % H) * P + i % P];
  U[i] = make_float2((a.x * b.x - a.y * b.y) * scale, (a.x * b.y + a.y * b.x) * scale);
}

__global__ void real_part_kernel(const float2* __restrict__ w, float* __restrict__ y, long long n) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = w[i].x;
}

inline dim3 grid_for(long long n) { return dim3((unsigned)((n + 255) / 256)); }

// Workspace layout of the 2-D circular convolution (complex64 elements):
// [B*H*P spectra of u][H*P spectra of k][stage scratch of B*H images].
inline long long circconv2d_elems(long long B, long long H, int N0, int N1) {
  const long long P = (long long)N0 * N1, t = work2_elems(B * H, N0, N1);
  if (t < 0) return -1;
  return (B * H + H) * P + t;
}

inline hipError_t circconv2d(const float* u, const float* k, float* y, float2* work, long long B, int H, int N0,
                             int N1, hipStream_t st) {
  const long long P = (long long)N0 * N1, nu = B * H * P, nk = (long long)H * P;
  float2 *U = work, *K = work + nu, *T = K + nk;
  hipLaunchKernelGGL(widen_kernel, grid_for(nu), dim3(256), 0, st, u, U, nu);
  hipLaunchKernelGGL(widen_kernel, grid_for(nk), dim3(256), 0, st, k, K, nk);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  if ((err = run2(U, U, T, B * H, N0, N1, 0, 1.f, st)) != hipSuccess) return err;
  if ((err = run2(K, K, T, H, N0, N1, 0, 1.f, st)) != hipSuccess) return err;
  hipLaunchKernelGGL(spectrum_product_kernel, grid_for(nu), dim3(256), 0, st, U, (const float2*)K, P, H, nu,
                     (float)(1.0 / (double)P));
  if ((err = hipGetLastError()) != hipSuccess) return err;
  if ((err = run2(U, U, T, B * H, N0, N1, 1, 1.f, st)) != hipSuccess) return err;
  hipLaunchKernelGGL(real_part_kernel, grid_for(nu), dim3(256), 0, st, (const float2*)U, y, nu);
  return hipGetLastError();
}

}  // namespace xf
}  // namespace sffft
