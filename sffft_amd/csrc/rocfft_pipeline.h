/* rocFFT comparator: the unfused FFT convolution pipeline the fused kernel is
 * measured against (the reference's cuFFT pipeline, src/sffft.cu:289-305,365-371):
 *   full = pad(u) -> R2C (N = 2L, batch B*H) -> U *= Kh[s mod H] -> C2R -> slice
 *   core = R2C -> multiply -> C2R
 * with Kh = DFT_N(pad(k))[0..N/2] / N prepared once by a C2C forward transform.
 * Not part of the drop-in boundary: measurement infrastructure for the driver. */
#ifndef SFFFT_ROCFFT_PIPELINE_H
#define SFFFT_ROCFFT_PIPELINE_H
#ifdef __cplusplus
extern "C" {
#endif

typedef struct sffft_rocfft sffft_rocfft;

/* Creates plans and work buffers for B*H sequences of length L (device memory is
 * owned by the handle). Returns 0 on success. */
int sffft_rocfft_create(int B, int H, int L, void* stream, sffft_rocfft** out);
/* Filter spectrum from k [H][L] fp32 (device): writes the unnormalised natural-order
 * spectrum Kc [H][2L] complex64 into kc (device, may be NULL) and keeps Kh inside. */
int sffft_rocfft_filter(sffft_rocfft* h, const float* k, void* kc);
/* Full pipeline u [B][H][L] fp32 -> y [B][H][L] fp32 (device). */
int sffft_rocfft_full(sffft_rocfft* h, const float* u, float* y);
/* Core only (R2C, multiply, C2R) on the handle's padded buffers. */
int sffft_rocfft_core(sffft_rocfft* h);
void sffft_rocfft_destroy(sffft_rocfft* h);

#ifdef __cplusplus
}
#endif
#endif
