/* oracle.c - CPU restatement of the reference's algorithm for the fused causal
 * long-convolution path. TEST INFRASTRUCTURE ONLY: it is the checker used by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, never part of
 * the product path (libsffft.so does not link or load it).
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the reference tree). How each function is pinned is stated next to it:
 *   oracle_ref_inputs       src/sffft.cu:308-310,339-341  pinned: bit-exact replay of
 *                           the xorshift64 stream checked in tests against an independent
 *                           numpy restatement and the published per-plan error scale.
 *   oracle_direct_conv      src/sffft.cu:375-378          pinned: closed forms (delta filter
 *                           = shifted copy, box filter = prefix sums), brute force, np.convolve.
 *   oracle_fft_conv         (fp64 FFT convolution)        pinned: against oracle_direct_conv.
 *   oracle_spectrum_p_order src/sffft.cu:283-288,342-344,365  pinned: numpy.fft on the
 *                           digit permutation (closed form of permuteK).
 *   oracle_fourstep_conv    Appendix-A schedule of src/sffft.cu:137-241,273-279 in fp64
 *                           pinned: equals the direct convolution to ~1e-14 for every plan.
 *   oracle_fourstep_fp16    same schedule with fp16 rounding of storage, operands, and
 *                           (optionally) the raw accumulator; pinned: fp64 mode of the same
 *                           code equals oracle_fourstep_conv; mode 1 and mode 2 reproduce the
 *                           published fp32- and fp16-accumulation errors per plan
 *                           (results/gb10_allocator_sweep.csv) within 25%; mode 2 overflows to
 *                           inf/nan at input scale 15000 where mode 1 stays within 1e-3, as
 *                           tests/precision_smoke.sh:49-56 requires of the kernels.
 *   oracle_select_candidate src/selection.h:13-24         pinned: tests/selection_test.cpp
 *   oracle_relative_l2      src/selection.h:26-29         asserts + the reference header
 *                           compiled from the reference tree (oracle/_ref).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifndef M_PI
#define M_PI 3.14159265358979323846
#endif

/* ---- reference input generator (src/sffft.cu:308-310, 339-341) ------------- */
typedef struct { uint64_t s; } xs64;
static double urand(xs64* r) {
  r->s ^= r->s << 13;
  r->s ^= r->s >> 7;
  r->s ^= r->s << 17;
  return ((double)(r->s >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}
/* The two urand() calls of `sqrt(-2*log(urand()))*cos(2*M_PI*urand())` are
 * unsequenced in C++; GCC and clang evaluate the log argument first. */
static double nrand(xs64* r) {
  const double u1 = urand(r);
  const double u2 = urand(r);
  return sqrt(-2 * log(u1)) * cos(2 * M_PI * u2);
}

/* u[b][h][n] = (float)(nrand()*scale) in (b,h,n) order, then
 * k[h][n] = (float)(nrand()*exp(-a n)*sqrt(2a)), a = 1/(4 + L h / H). */
void oracle_ref_inputs(uint64_t seed, int B, int H, int L, double input_scale, float* u, float* k) {
  xs64 r = {seed};
  const size_t n = (size_t)B * H * L;
  for (size_t i = 0; i < n; i++) u[i] = (float)(nrand(&r) * input_scale);
  for (int h = 0; h < H; h++) {
    const double a = 1.0 / (4.0 + (double)L * h / H);
    for (int t = 0; t < L; t++) k[(size_t)h * L + t] = (float)(nrand(&r) * exp(-a * t) * sqrt(2 * a));
  }
}

/* ---- fp64 direct causal convolution (src/sffft.cu:376-377) ------------------- */
typedef struct {
  const float *u, *k;
  double* y;
  int B, H, L;
  size_t s0, s1;
} conv_job;

static void* direct_worker(void* p) {
  conv_job* j = (conv_job*)p;
  for (size_t s = j->s0; s < j->s1; s++) {
    const int h = (int)(s % (size_t)j->H);
    const float* us = j->u + s * j->L;
    const float* kh = j->k + (size_t)h * j->L;
    double* ys = j->y + s * j->L;
    for (int n = 0; n < j->L; n++) {
      double acc = 0;
      for (int m = 0; m <= n; m++) acc += (double)us[m] * kh[n - m];
      ys[n] = acc;
    }
  }
  return 0;
}

/* Sequences are s = b*H + h; k row is h = s mod H. Splits sequences over threads. */
void oracle_direct_conv(const float* u, const float* k, double* y, int B, int H, int L, int nthreads) {
  const size_t S = (size_t)B * H;
  if (nthreads < 1) nthreads = 1;
  if ((size_t)nthreads > S) nthreads = (int)S;
  pthread_t th[256];
  conv_job jobs[256];
  if (nthreads > 256) nthreads = 256;
  for (int t = 0; t < nthreads; t++) {
    jobs[t] = (conv_job){u, k, y, B, H, L, S * t / nthreads, S * (t + 1) / nthreads};
    if (nthreads == 1)
      direct_worker(&jobs[t]);
    else
      pthread_create(&th[t], 0, direct_worker, &jobs[t]);
  }
  if (nthreads > 1)
    for (int t = 0; t < nthreads; t++) pthread_join(th[t], 0);
}

/* Sampled sequences only (src/sffft.cu:376: {0, BH/2, BH-1}); seqs[i] are s indices. */
void oracle_direct_conv_seqs(const float* u, const float* k, double* y, int H, int L, const int64_t* seqs,
                             int nseq) {
  for (int i = 0; i < nseq; i++) {
    conv_job j = {u + (size_t)seqs[i] * L, k, y + (size_t)i * L, 1, H, L, 0, 1};
    /* sequence row is passed pre-offset; its channel is seqs[i] mod H */
    const int h = (int)(seqs[i] % H);
    j.k = k + (size_t)h * L;
    j.H = 1;
    direct_worker(&j);
  }
}

/* ---- fp64 FFT (iterative radix-2, natural order in and out) ----------------- */
static void fft64(double* re, double* im, int n, int inverse) {
  for (int i = 1, j = 0; i < n; i++) {
    int bit = n >> 1;
    for (; j & bit; bit >>= 1) j ^= bit;
    j ^= bit;
    if (i < j) {
      double t = re[i]; re[i] = re[j]; re[j] = t;
      t = im[i]; im[i] = im[j]; im[j] = t;
    }
  }
  for (int len = 2; len <= n; len <<= 1) {
    const double ang = (inverse ? 2 : -2) * M_PI / len;
    for (int i = 0; i < n; i += len)
      for (int j = 0; j < len / 2; j++) {
        const double wr = cos(ang * j), wi = sin(ang * j);
        const double xr = re[i + j + len / 2], xi = im[i + j + len / 2];
        const double tr = xr * wr - xi * wi, ti = xr * wi + xi * wr;
        re[i + j + len / 2] = re[i + j] - tr;
        im[i + j + len / 2] = im[i + j] - ti;
        re[i + j] += tr;
        im[i + j] += ti;
      }
  }
}

typedef struct {
  const float *u, *k;
  double* y;
  int H, L;
  size_t s0, s1;
} fft_job;

static void* fft_worker(void* p) {
  fft_job* j = (fft_job*)p;
  const int L = j->L, N = 2 * L;
  double* ur = (double*)malloc(sizeof(double) * N * 4);
  double *ui = ur + N, *kr = ur + 2 * N, *ki = ur + 3 * N;
  int last_h = -1;
  for (size_t s = j->s0; s < j->s1; s++) {
    const int h = (int)(s % (size_t)j->H);
    if (h != last_h) {
      for (int n = 0; n < N; n++) { kr[n] = n < L ? j->k[(size_t)h * L + n] : 0; ki[n] = 0; }
      fft64(kr, ki, N, 0);
      last_h = h;
    }
    for (int n = 0; n < N; n++) { ur[n] = n < L ? j->u[s * L + n] : 0; ui[n] = 0; }
    fft64(ur, ui, N, 0);
    for (int n = 0; n < N; n++) {
      const double a = ur[n] * kr[n] - ui[n] * ki[n], b = ur[n] * ki[n] + ui[n] * kr[n];
      ur[n] = a; ui[n] = b;
    }
    fft64(ur, ui, N, 1);
    for (int n = 0; n < L; n++) j->y[s * L + n] = ur[n] / N;
  }
  free(ur);
  return 0;
}

/* fp64 FFT convolution of every sequence (for lengths where O(L^2) is too slow). */
void oracle_fft_conv(const float* u, const float* k, double* y, int B, int H, int L, int nthreads) {
  const size_t S = (size_t)B * H;
  if (nthreads < 1) nthreads = 1;
  if (nthreads > 256) nthreads = 256;
  if ((size_t)nthreads > S) nthreads = (int)S;
  pthread_t th[256];
  fft_job jobs[256];
  /* sequences s = b*H + h: give each thread whole ranges; channel FFTs are cached per run of equal h */
  for (int t = 0; t < nthreads; t++) {
    jobs[t] = (fft_job){u, k, y, H, L, S * t / nthreads, S * (t + 1) / nthreads};
    if (nthreads == 1)
      fft_worker(&jobs[t]);
    else
      pthread_create(&th[t], 0, fft_worker, &jobs[t]);
  }
  if (nthreads > 1)
    for (int t = 0; t < nthreads; t++) pthread_join(th[t], 0);
}

/* ---- digit order (src/sffft.cu:283-288) --------------------------------------- */
/* p = d0*(R1*R2) + d1*R2 + d2  holds frequency f = d0 + R0*d1 + R0*R1*d2. */
static int p_to_freq(int p, int r0, int r1, int r2) {
  const int d2 = p % r2, d1 = (p / r2) % r1, d0 = p / (r1 * r2);
  return d0 + r0 * (d1 + r1 * d2);
}

/* Unnormalised spectrum of the zero-padded filter row in digit order (p-order):
 * out[2p], out[2p+1] = Re, Im of DFT_N(pad(k))[p_to_freq(p)]. */
void oracle_spectrum_p_order(const float* k, int L, int r0, int r1, int r2, double* out) {
  const int N = 2 * L;
  double* re = (double*)malloc(sizeof(double) * N * 2);
  double* im = re + N;
  for (int n = 0; n < N; n++) { re[n] = n < L ? k[n] : 0; im[n] = 0; }
  fft64(re, im, N, 0);
  for (int p = 0; p < N; p++) {
    const int f = p_to_freq(p, r0, r1, r2);
    out[2 * p] = re[f];
    out[2 * p + 1] = im[f];
  }
  free(re);
}

/* ---- the four-step schedule, fp64 or fp16-rounded ------------------------------
 * Restates left_stage/right_stage/fftconv (src/sffft.cu:137-241, 266-279) and the
 * twiddle exponent twid<P,J> (src/sffft.cu:106-113) on natural positions p:
 *   forward  J = 0..S-1:  X <- (F_R/sqrt R) along digit J; then X[p] *= w^{e_J(p)}
 *                         (J < S-1) or X[p] *= Kf[p] (J = S-1)
 *   inverse  J = S-1..0:  X <- (conj F_R/sqrt R) along digit J; then X[p] *= conj w^{e_{J-1}(p)}
 *                         (J > 0) or y[p] = Re X[p] for p < L (J = 0)
 * mode 0: fp64 throughout. mode 1: fp16 emulation of the fused kernel: input,
 * DFT coefficients and every stage output stored as fp16 (round to nearest even),
 * twiddles, scales and spectrum in fp32-equivalent double. mode 2: mode 1 plus the
 * raw (unscaled) stage accumulator rounded to fp16 (fp16-accumulation mode). */
static double round_f16(double x) {
  if (isnan(x)) return x;
  const double ax = fabs(x);
  if (ax >= 65520.0) return x > 0 ? INFINITY : -INFINITY;
  if (ax < 6.103515625e-05) { /* subnormal: quantum 2^-24 */
    const double q = 5.9604644775390625e-08;
    return nearbyint(x / q) * q;
  }
  int e;
  frexp(ax, &e); /* ax = f * 2^e, f in [0.5, 1) */
  const double q = ldexp(1.0, e - 11);
  return nearbyint(x / q) * q; /* nearbyint: ties to even in the default rounding mode */
}
static double round_f32(double x) { return (double)(float)x; }
double oracle_round_f16(double x) { return round_f16(x); }

static int digit_stride(int J, int r1, int r2) { return J == 0 ? r1 * r2 : J == 1 ? r2 : 1; }
static int twid_exp(int p, int J, int N, int r0, int r1, int r2) {
  const int R[3] = {r0, r1, r2};
  const int Nm = J == 0 ? N : J == 1 ? N / r0 : N / (r0 * r1);
  const int Nm1 = digit_stride(J, r1, r2);
  const int nrest = p % Nm1, km = (p / Nm1) % R[J];
  return (N / Nm) * nrest * km; /* e in [0, N) */
}

/* x: real input (L), kf: p-order spectrum (2N doubles, unnormalised), y: L outputs. */
void oracle_fourstep_conv(const double* x, const double* kf, int L, int r0, int r1, int r2, int mode, double* y) {
  const int N = 2 * L, S = r2 > 1 ? 3 : 2;
  const int R[3] = {r0, r1, r2 > 1 ? r2 : 1};
  double* Xr = (double*)malloc(sizeof(double) * N * 4);
  double *Xi = Xr + N, *Tr = Xr + 2 * N, *Ti = Xr + 3 * N;
  const int q = mode >= 1;
  for (int n = 0; n < N; n++) { Xr[n] = n < L ? (q ? round_f16(x[n]) : x[n]) : 0; Xi[n] = 0; }
  for (int pass = 0; pass < 2 * S; pass++) {
    const int inv = pass >= S, J = inv ? 2 * S - 1 - pass : pass;
    const int Rj = R[J], s = digit_stride(J, r1, r2);
    const double sc = 1.0 / sqrt((double)Rj);
    for (int p = 0; p < N; p++) {
      const int outer = p / (Rj * s), dig = (p / s) % Rj, inner = p % s;
      double ar = 0, ai = 0;
      for (int t = 0; t < Rj; t++) {
        const int pt = outer * Rj * s + t * s + inner;
        const int e = (dig * t) % Rj;
        double c = cos(2 * M_PI * e / Rj), sn = -sin(2 * M_PI * e / Rj); /* F = c + i sn */
        if (q) { c = round_f16((double)(float)c); sn = round_f16((double)(float)sn); }
        if (inv) sn = -sn;
        ar += c * Xr[pt] - sn * Xi[pt];
        ai += c * Xi[pt] + sn * Xr[pt];
      }
      if (mode == 2) { ar = round_f16(ar); ai = round_f16(ai); }
      ar *= sc;
      ai *= sc;
      double wr, wi;
      if (!inv && J == S - 1) {
        wr = kf[2 * p]; wi = kf[2 * p + 1];
        if (q) { wr = round_f32(wr); wi = round_f32(wi); }
      } else if (!inv) {
        const int e = twid_exp(p, J, N, r0, r1, r2);
        wr = cos(2 * M_PI * e / N); wi = -sin(2 * M_PI * e / N);
      } else if (J > 0) {
        const int e = twid_exp(p, J - 1, N, r0, r1, r2);
        wr = cos(2 * M_PI * e / N); wi = sin(2 * M_PI * e / N);
      } else {
        wr = 1; wi = 0;
      }
      double orr = ar * wr - ai * wi, oi = ar * wi + ai * wr;
      if (q && !(inv && J == 0)) { orr = round_f16(orr); oi = round_f16(oi); }
      Tr[p] = orr;
      Ti[p] = oi;
    }
    memcpy(Xr, Tr, sizeof(double) * N);
    memcpy(Xi, Ti, sizeof(double) * N);
  }
  for (int n = 0; n < L; n++) y[n] = Xr[n];
  free(Xr);
}

/* ---- selector and error (src/selection.h:13-29) -------------------------------- */
typedef struct {
  const char* method;
  const char* io;
  const char* config;
  double ms, rel_err;
} oracle_candidate;

int oracle_select_candidate(const oracle_candidate* c, int n, double max_error, const char* io) {
  if (!isfinite(max_error) || max_error <= 0) return -1;
  if (strcmp(io, "fp32") && strcmp(io, "bf16") && strcmp(io, "any")) return -1;
  int best = -1;
  for (int i = 0; i < n; i++) {
    if (strcmp(io, "any") && strcmp(io, c[i].io)) continue;
    if (!isfinite(c[i].ms) || c[i].ms <= 0 || !isfinite(c[i].rel_err) || c[i].rel_err < 0 ||
        c[i].rel_err > max_error)
      continue;
    if (best < 0 || c[i].ms < c[best].ms || (c[i].ms == c[best].ms && c[i].rel_err < c[best].rel_err)) best = i;
  }
  return best;
}

double oracle_relative_l2(double squared_error, double squared_reference) {
  if (squared_reference > 0) return sqrt(squared_error / squared_reference);
  return squared_error == 0 ? 0 : INFINITY;
}
