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
// the last stage writes each value to its natural-order slot directly.
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
  // The line's DFT in registers: radix-2 decimation in frequency over log2(R) levels,
  // natural input order, bit-reversed output order; fp64, twiddles w_R^e from the table.
  // About R*log2(R)/2 complex products instead of the R*R of the dense sum.
  double vr[R], vi[R];
#pragma unroll
  for (int t = 0; t < R; t++) {
    vr[t] = (double)x[t].x;
    vi[t] = (double)x[t].y;
  }
#pragma unroll
  for (int m = R; m >= 2; m >>= 1) {
    const int h = m >> 1, step = R / m;  // w_m^j = w_R^(j * step)
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
          vr[i1] = dr * c - di * sn;
          vi[i1] = dr * sn + di * c;
        }
      }
  }
  auto bitrev = [](int k) {
    int r = 0;
#pragma unroll
    for (int b = 1; b < R; b <<= 1) r = (r << 1) | ((k & b) ? 1 : 0);
    return r;
  };
  if (last) {
#pragma unroll
    for (int k = 0; k < R; k++) {
      const int r = bitrev(k);
      dst[(kbase + (long long)k * wlast) * q.stride] = make_float2((float)(vr[r] * scale), (float)(vi[r] * scale));
    }
  } else {
    // twiddle w_Nj^(k * inner) before the next stage: powers of w_Nj^inner, in fp64
    double w1s, w1c;
    sincospi(2.0 * (double)inner / (double)Nj, &w1s, &w1c);
    w1s *= sign;
    double wr = 1.0, wi = 0.0;
#pragma unroll
    for (int k = 0; k < R; k++) {
      const int r = bitrev(k);
      work[widx(base + k * sJ)] =
          make_float2((float)(vr[r] * wr - vi[r] * wi), (float)(vr[r] * wi + vi[r] * wr));
      const double nr = wr * w1c - wi * w1s;
      wi = wr * w1s + wi * w1c;
      wr = nr;
    }
  }
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
