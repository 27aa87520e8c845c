/* sffft.h - C ABI of the MI355X fused causal long-convolution library (libsffft.so).
 *
 *   y[b,h,n] = sum_{m<=n} u[b,h,m] * k[h,n-m],  n < L,  L a power of two in [128, 16384]
 *   (single-pass plans) or in [2048, 131072] (multi-pass plans, sffft_conv_long_*)
 *
 * The reference has no library: its interface is two kernel launches inside
 * src/sffft.cu. Each entry point below names the reference code it replaces.
 *
 * Conventions
 *  - All pointers are device pointers (hipMalloc'd) unless stated otherwise.
 *    u and y are [B][H][L] row-major; k is [H][L]; rows must be 16-byte aligned.
 *  - `stream` is a hipStream_t (NULL = default stream). Calls are asynchronous on
 *    that stream, reentrant, and allocate no memory, except that the first call on a
 *    device uploads an immutable 57,344-byte DFT coefficient table, and the first
 *    mode-1 call of a plan its twiddle table (kept for the life of the process).
 *  - Every function returns SFFFT_OK (0) or a positive error code; nothing exits.
 */
#ifndef SFFFT_H
#define SFFFT_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SFFFT_OK 0
#define SFFFT_EINVAL 1      /* invalid argument (sizes, plan, null pointer, misalignment) */
#define SFFFT_ENOPLAN 2     /* the plan is valid but was not compiled into this library */
#define SFFFT_EHIP 3        /* the HIP runtime reported an error */
#define SFFFT_ENOTFOUND 4   /* no candidate/plan matches the request */
#define SFFFT_ESCRATCH 5    /* more workspace than sffft_spectrum_noalloc's static scratch */

/* A transform plan: N = 2L = r0*r1*r2 (r2 = 1 for two-stage plans), radices in
 * {16,32,64}. Mirrors Plan<R0,R1,R2> and the W template argument of fftconv
 * (src/sffft.cu:92-104, 243-245, 507-513).
 *   waves : wavefronts (64 lanes) per workgroup
 *   acc   : 0 = fp32 accumulation, 1 = fp16 accumulation ("fp16acc" methods)
 *   cached: 1 = DFT matrices from the coefficient table ("kernel_cached"),
 *           0 = computed in the kernel ("kernel_legacy")  (src/sffft.cu:253-265)
 *   seqs  : sequences per transform: 1, or 2 (two batch rows of one channel packed
 *           as the real and imaginary parts of one complex transform; B must be even)
 *   mode  : 0 = one workgroup per transform, stages exchanged through LDS;
 *           1 = one wavefront per transform, stages chained in registers, `waves`
 *               wavefronts per workgroup sharing LDS-resident DFT and twiddle tables
 *               (two-stage plans, seqs = 2; the first call for such a plan on a device
 *               uploads its immutable twiddle tables, 32*L bytes; 16*L for acc = 1)
 *   channels : mode 1 only: channels per workgroup; their spectra are copied into
 *           LDS once and shared by the wavefronts of each channel (mode 0: 1)
 *   mode 2 : multi-pass (sffft_conv_long_*): N = r0 * (r1 * r2), a column transform of
 *           radix r0 and row transforms of length r1*r2 (the wave pipeline's two-stage
 *           row plan), with the intermediate in a caller-provided workspace; waves = 4,
 *           acc = 0, cached = 1, seqs = 2, channels = 1
 */
typedef struct sffft_plan {
  int r0, r1, r2;
  int waves;
  int acc;
  int cached;
  int seqs;
  int mode;
  int channels;
} sffft_plan;

/* Plan validity: SFFFT_OK, SFFFT_EINVAL (bad radices/product/LDS), SFFFT_ENOPLAN.
 * Replaces the host check `if (P::L != L)` (src/sffft.cu:383). */
int sffft_plan_check(int L, const sffft_plan* plan);

/* LDS bytes per workgroup (Plan::smem<W,TAcc>(), src/sffft.cu:103). 0 if invalid. */
size_t sffft_plan_lds_bytes(int L, const sffft_plan* plan);

/* Workgroups of this plan resident per CU (cudaOccupancyMaxActiveBlocksPerMultiprocessor,
 * src/sffft.cu:388). Requires a HIP device. */
int sffft_plan_occupancy(int L, const sffft_plan* plan, int* blocks_per_cu);

/* The plan registry used by the driver and the selector: the i-th compiled plan
 * for length L (acc = 0, cached = 1 are filled in; callers vary them; r*, waves,
 * seqs and mode identify the compiled kernel). For L > 16384 it lists the compiled
 * multi-pass (mode 2) plans. Writes the plan name ("64x32") into
 * name. Returns SFFFT_ENOTFOUND past the end.
 * Replaces the RUN(...) plan table (src/sffft.cu:506-513). */
int sffft_plan_count(int L);
int sffft_plan_get(int L, int index, sffft_plan* plan, char* name, size_t name_len);

/* Bytes of the kernel-order filter spectrum: H * 2L * 8 (complex64). */
size_t sffft_spectrum_bytes(int H, int L);

/* Filter spectrum in the fused kernel's order, from the real filter k [H][L] fp32, as
 * kf [H][2L] complex64: row h holds channel h's spectrum for every plan, so rows of
 * spectra may be sliced and concatenated along the channels. The order within a row
 * depends on the radices and on the mode (mode 0 and mode 1 differ). For mode-1 (wave)
 * plans only the Hermitian half is stored (K[2L-f] = conj(K[f]) for a real filter):
 * (r0/2 + 1) * (8*(r1/16) + 1) * 2 complex64 values at the start of each row, the rest of
 * the row zero.
 * `work` must hold sffft_spectrum_bytes(H, L) bytes (scratch, clobbered).
 * Replaces: zero-pad + cufftExecC2C(FORWARD) + permuteK (src/sffft.cu:342-344,365,384,283-288).
 * Arithmetic: fp64 accumulation and twiddles, fp32 storage between the stages. */
int sffft_spectrum(const float* k, int H, int L, const sffft_plan* plan, void* kf, void* work, void* stream);

/* sffft_spectrum of the conjugate spectrum conj(K), same layout and arguments. No counterpart
 * in the reference: it serves the gradients of the convolution. With the 2L zero padding the
 * anti-causal correlation z[m] = sum_{n>=m} x[n] k[n-m] (m < L), which the input and filter
 * gradients are, is sffft_conv_* of x with this spectrum: no time reversal of x or z. */
int sffft_spectrum_conj(const float* k, int H, int L, const sffft_plan* plan, void* kf, void* work, void* stream);

/* sffft_spectrum without the `work` argument, for callers that cannot allocate (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. It stages the channels through a static device array of 32 MiB per GPU (held
 * until the process ends; 2L*8 bytes per channel, so the channels run in chunks) and calls
 * no hipMalloc, hipFree or allocating routine; its output is bit-identical to
 * sffft_spectrum's. Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (two streams, two host threads) race. SFFFT_ESCRATCH if one channel needs more than
 * the array (never for a valid L). */
int sffft_spectrum_noalloc(const float* k, int H, int L, const sffft_plan* plan, void* kf, void* stream);

/* Complex input: the spectrum of the complex filter kr + i*ki (kr, ki [H][L] fp32) for a plan
 * with two sequences per transform (seqs = 2; every mode-1 and mode-2 plan). With it,
 * sffft_conv_complex_* (and sffft_conv_long_* for mode-2 plans) compute the complex causal
 * convolution
 *   y[b] + i y[b+1] = sum_{m<=n} (u[b,m] + i u[b+1,m]) (kr[n-m] + i ki[n-m])
 * for every even b: batch rows 2b' and 2b'+1 of u and y are the real and imaginary planes of
 * complex sequence b'. The reference takes real input only (README.md:174); no counterpart.
 * `work` as in sffft_spectrum; kf holds the sum of both spectra, whole (not Hermitian). */
int sffft_spectrum_complex(const float* kr, const float* ki, int H, int L, const sffft_plan* plan, void* kf,
                           void* work, void* stream);

/* sffft_spectrum from an unnormalised natural-order spectrum kc [H][2L] complex64
 * (kc[h][f] = sum_n k[h][n] exp(-2 pi i f n / 2L), e.g. from hipFFT C2C) of a REAL filter k:
 * for mode-1 plans only the Hermitian half of kc is read (frequencies above L are taken as
 * the conjugates of their partners 2L - f), so kc must be the spectrum of a real filter.
 * Replaces permuteK (src/sffft.cu:283-288). kc and kf must not overlap. */
int sffft_spectrum_from_natural(const void* kc, int H, int L, const sffft_plan* plan, void* kf, void* stream);

/* The same gather for any spectrum kc, e.g. of a complex filter kr + i*ki: every frequency
 * is read and the whole spectrum stored, the layout sffft_spectrum_complex writes, for
 * sffft_conv_complex_* (and sffft_conv_long_*). Plans with two sequences per transform
 * (seqs = 2). No counterpart in the reference (real filters only, README.md:174). */
int sffft_spectrum_from_natural_complex(const void* kc, int H, int L, const sffft_plan* plan, void* kf,
                                        void* stream);

/* The fused convolution, one launch: grid = H*B/seqs workgroups of 64*waves lanes
 * (mode 0) or ceil(H / channels) workgroups of 64*waves lanes (mode 1).
 * Replaces fftconv<P,W,float|bf16,TAcc,CACHED><<<B*H, 32*W, smem>>> (src/sffft.cu:243-280,389-390).
 * kf must come from sffft_spectrum* with the same L and the same r0/r1/r2. */
int sffft_conv_f32(const float* u, const void* kf, float* y, int B, int H, int L, const sffft_plan* plan,
                   void* stream);
/* bf16 I/O: u and y hold bf16 bit patterns; y is rounded to nearest even. */
int sffft_conv_bf16(const uint16_t* u, const void* kf, uint16_t* y, int B, int H, int L,
                    const sffft_plan* plan, void* stream);

/* Complex causal convolution with a spectrum from sffft_spectrum_complex (see there):
 * seqs = 2 plans of modes 0 and 1, fp32 accumulation; the same launch shape as
 * sffft_conv_*. No counterpart in the reference (real input only, README.md:174). */
int sffft_conv_complex_f32(const float* u, const void* kf, float* y, int B, int H, int L,
                           const sffft_plan* plan, void* stream);
int sffft_conv_complex_bf16(const uint16_t* u, const void* kf, uint16_t* y, int B, int H, int L,
                            const sffft_plan* plan, void* stream);

/* Multi-pass convolution (mode-2 plans), for sequences whose length-2L transform does
 * not fit one CU's LDS. No counterpart in the reference, which stops at L = 8192 and
 * names a four-step split with an HBM pass as the way beyond (README.md:175). Three
 * launches on `stream` per chunk of channels: a column transform of radix r0 over the
 * input, the row transforms with the spectrum product, and the inverse column transform.
 * `work` is caller-owned device memory (the complex fp16 intermediate), 16-byte aligned
 * and disjoint from u, y and kf, of work_bytes >= (B/2) * 2L * 4 bytes (one channel);
 * the batch runs in chunks of floor(work_bytes / that) channels and the contents are
 * clobbered. kf comes from sffft_spectrum* with the same plan. B must be even (pairs of
 * sequences). Same error codes as sffft_conv_*. */
/* The default workspace: chunks of at most 96 MiB, which stay in the 256 MB Infinity
 * Cache between the passes (the whole batch if smaller). 0 if invalid or not mode 2. */
size_t sffft_work_bytes(int B, int H, int L, const sffft_plan* plan);
int sffft_conv_long_f32(const float* u, const void* kf, float* y, void* work, size_t work_bytes, int B, int H, int L,
                        const sffft_plan* plan, void* stream);
int sffft_conv_long_bf16(const uint16_t* u, const void* kf, uint16_t* y, void* work, size_t work_bytes, int B, int H,
                         int L, const sffft_plan* plan, void* stream);

/* Circular (non-causal) convolution of period N with a multi-pass plan (r0*r1*r2 = N):
 *   y[b,h,n] = sum_{m<N} u[b,h,m] * k[h,(n-m) mod N],  n < N,
 * u, y [B][H][N], k [H][N]. The reference lists non-causal and circular convolution as not
 * exposed (README.md:174); no counterpart. The same passes as sffft_conv_long_* over rows of
 * length N with no zero half; the spectrum is the DFT of the unpadded filter
 * (sffft_spectrum_circular, same order as sffft_spectrum for the plan, H*N*8 bytes, `work`
 * as in sffft_spectrum). Workspace: sffft_work_bytes(B, H, N/2, plan) (same chunking). */
int sffft_spectrum_circular(const float* k, int H, int N, const sffft_plan* plan, void* kf, void* work,
                            void* stream);
int sffft_circconv_long_f32(const float* u, const void* kf, float* y, void* work, size_t work_bytes, int B, int H,
                            int N, const sffft_plan* plan, void* stream);
int sffft_circconv_long_bf16(const uint16_t* u, const void* kf, uint16_t* y, void* work, size_t work_bytes, int B,
                             int H, int N, const sffft_plan* plan, void* stream);

/* Standalone complex transforms. The reference lists standalone forward/inverse FFTs and
 * 2-D convolution as not exposed (README.md:174); no counterpart. Complex64 in and out,
 * unnormalised:
 *   X[b,k] = scale * sum_{n<N} x[b,n] * exp(-/+ 2 pi i n k / N)
 * with the minus sign for inverse = 0 and the plus sign for inverse = 1. N is a power of two
 * in [2, 2^24] and batch * N <= 2^31. Element n of sequence b sits at x[b * dist + n * stride]
 * (complex elements, stride >= 1, dist >= 1 when batch > 1); X has the same layout and may
 * equal x. Two layout families are supported: whole sequences one after another
 * (dist >= N * stride) and sequences interleaved within one element step
 * (stride >= batch * dist, as the columns of a row-major matrix); other layouts, even
 * non-overlapping ones, are rejected with SFFFT_EINVAL. `work` holds sffft_fft_work_bytes(batch, N) bytes (NULL allowed when that is 0) and
 * must not overlap x or X. Each stage is a radix-<=64 DFT evaluated in fp64 and stored as
 * complex64 (relative error ~1e-7); pointers 8-byte aligned. sffft_fft_work_bytes returns 0
 * for sizes the call rejects. */
size_t sffft_fft_work_bytes(int batch, int N);
int sffft_fft_c2c(const void* x, void* X, void* work, size_t work_bytes, int batch, int N, long long stride,
                  long long dist, int inverse, float scale, void* stream);

/* 2-D transform of `batch` contiguous [N0][N1] complex64 arrays (every row, then every
 * column), same sign, scale, size and aliasing rules as sffft_fft_c2c per axis, and
 * batch * N0 * N1 <= 2^31. `work`: sffft_fft2_work_bytes(batch, N0, N1) bytes. */
size_t sffft_fft2_work_bytes(int batch, int N0, int N1);
int sffft_fft2_c2c(const void* x, void* X, void* work, size_t work_bytes, int batch, int N0, int N1, int inverse,
                   float scale, void* stream);

/* 2-D circular convolution of period (N0, N1), fp32 in and out:
 *   y[b,h,i,j] = sum_{a<N0, c<N1} u[b,h,a,c] * k[h,(i-a) mod N0,(j-c) mod N1]
 * u, y [B][H][N0][N1], k [H][N0][N1], through 2-D transforms as sffft_fft2_c2c (complex
 * spectrum product, inverse, real part). `work` holds sffft_circconv2d_work_bytes(B, H, N0,
 * N1) bytes and must not overlap u, k or y; y may not overlap u or k. */
size_t sffft_circconv2d_work_bytes(int B, int H, int N0, int N1);
int sffft_circconv2d_f32(const float* u, const float* k, float* y, void* work, size_t work_bytes, int B, int H,
                         int N0, int N1, void* stream);

/* fp32 -> bf16 (round to nearest even) on the device. Replaces tobf16 (src/sffft.cu:306). */
int sffft_to_bf16(const float* x, uint16_t* y, size_t n, void* stream);

/* Launches a body-less kernel with the grid, block and LDS size that sffft_conv_*
   uses for this plan and shape: timed back to back, it gives the dispatch floor of
   that launch shape. No counterpart in the reference (a measurement aid); same
   argument checks and error codes as sffft_conv_*, without the buffers. */
int sffft_dispatch_floor(int B, int H, int L, const sffft_plan* plan, void* stream);

/* The same body-less kernel with an explicit launch shape: grid workgroups of block lanes
   (a multiple of 64, at most 1024) requesting lds_bytes of LDS (at most 163840), to
   measure which part of the dispatch floor a launch shape controls. No counterpart in
   the reference (a measurement aid). SFFFT_EINVAL for a shape outside those limits. */
int sffft_dispatch_floor_shape(unsigned grid, unsigned block, unsigned lds_bytes, void* stream);

/* Copies the device DFT coefficient table (57,344 bytes) to host memory `out`
 * (for tests). Returns SFFFT_EINVAL if out_len is too small. */
int sffft_dft_table(void* out, size_t out_len);

/* Test probes of the twiddle factors (no counterpart in the reference; the reference's
 * twid(), src/sffft.cu:106-113, evaluates them with __sincosf in the kernel).
 * sffft_twiddle_probe evaluates on the device, with the workgroup kernel's own code
 * (v_sin/v_cos of the angle in revolutions plus complex recurrences), for each of the nq
 * queries (e0, step, f0, fstep) (device int[4] each): the four values
 * sc * exp(-2 pi i (e0 + step*v) / N), v = 0..3, and `rows` (<= 64) row steps, each the
 * product with exp(-2 pi i (f0 + fstep*v) / N); out is device complex64 [nq][rows+1][4].
 * N a power of two in [256, 32768]. sffft_twiddle_table copies the wave pipeline's twiddle
 * tables of plan r0 x r1 (built in fp64 on the host) to host memory `out`: layout 1 = fp32
 * split (the wave kernels'), 0 = fp32 paired (64x64 and the multi-pass row pass), r0*r1*16
 * bytes; 2 = fp16 (the wave kernels of the fp16-accumulation mode), r0*r1*8 bytes. */
int sffft_twiddle_probe(int N, const void* queries, int nq, int rows, float sc, void* out, void* stream);
int sffft_twiddle_table(int r0, int r1, int layout, void* out, size_t out_len);

/* Host-side selector (src/selection.h:8-29). A candidate is (method, io, config, ms,
 * rel_err); io is "fp32" or "bf16". Returns the index of the fastest candidate whose io
 * matches (io "any" matches both), with finite ms > 0 and finite 0 <= rel_err <=
 * max_error, ties on ms going to the lower rel_err; -1 if none or if max_error is not
 * positive and finite or io is unknown. */
typedef struct sffft_candidate {
  const char* method;
  const char* io;
  const char* config;
  double ms;
  double rel_err;
} sffft_candidate;
int sffft_select_candidate(const sffft_candidate* candidates, int n, double max_error, const char* io);

/* sqrt(squared_error / squared_reference); a zero reference gives 0 for a zero
 * error and +inf otherwise (src/selection.h:26-29). */
double sffft_relative_l2(double squared_error, double squared_reference);

const char* sffft_strerror(int code);

/* Text of the last HIP error recorded by a call on this thread ("" if none). */
const char* sffft_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* SFFFT_H */
