// Instantiates the fused kernels for every plan of one length (compiled once per
// length with -DSFFFT_INST_L=<L>, so the lengths build in parallel).
#include "fftconv.hpp"
#include "fftconv_wave.hpp"
#include "registry.hpp"

#ifndef SFFFT_INST_L
#error "compile with -DSFFFT_INST_L=<length>"
#endif

namespace sffft {

// Register budget of a workgroup-kernel plan (wavefronts per SIMD the allocation must
// allow; 1: the compiler's own). 64x16x16 with 8 wavefronts and table fragments is held
// to the occupancy its 80 KB of LDS allows (two workgroups per CU, 128 VGPRs): left
// alone it takes 147-156 VGPRs and loses a workgroup per CU (measured 10% slower). Held
// to their LDS-limited occupancy the other plans (and this one with in-kernel
// fragments) spill, or gain nothing.
template <class P, int NW, bool CACHED>
constexpr int fused_wpe() {
  return CACHED && P::R0 == 64 && P::R1 == 16 && P::R2 == 16 && NW == 8 ? lds_waves_per_simd<P, NW>() : 1;
}

template <class P, int NW, int NSEQ, class TIO, bool CACHED>
static hipError_t launch_fused(const void* u, const void* kf, void* y, int B, int H, const void* ftab, const void*,
                               int acc16, hipStream_t stream) {
  const unsigned grid = (unsigned)(H * (B / NSEQ));
  constexpr int WPE = fused_wpe<P, NW, CACHED>();
  if (acc16)
    hipLaunchKernelGGL((fftconv_kernel<P, NW, NSEQ, TIO, CACHED, true, WPE>), dim3(grid), dim3(64 * NW), 0, stream,
                       static_cast<const TIO*>(u), static_cast<const float2*>(kf), static_cast<TIO*>(y), B, H,
                       static_cast<const h8*>(ftab));
  else
    hipLaunchKernelGGL((fftconv_kernel<P, NW, NSEQ, TIO, CACHED, false, WPE>), dim3(grid), dim3(64 * NW), 0, stream,
                       static_cast<const TIO*>(u), static_cast<const float2*>(kf), static_cast<TIO*>(y), B, H,
                       static_cast<const h8*>(ftab));
  return hipGetLastError();
}

template <class P, int NW, int CH, class TIO, bool CACHED>
static hipError_t launch_wave(const void* u, const void* kf, void* y, int B, int H, const void* ftab,
                              const void* tw, int acc16, hipStream_t stream) {
  const unsigned grid = (unsigned)((H + CH - 1) / CH);
  if (acc16)
    hipLaunchKernelGGL((fftconv_wave_kernel<P, NW, CH, TIO, CACHED, true, true>), dim3(grid), dim3(64 * NW), 0,
                       stream, static_cast<const TIO*>(u), static_cast<const float4*>(kf), static_cast<TIO*>(y), B,
                       H, static_cast<const h8*>(ftab), static_cast<const float4*>(tw));
  else
    hipLaunchKernelGGL((fftconv_wave_kernel<P, NW, CH, TIO, CACHED, false, true>), dim3(grid), dim3(64 * NW), 0,
                       stream, static_cast<const TIO*>(u), static_cast<const float4*>(kf), static_cast<TIO*>(y), B,
                       H, static_cast<const h8*>(ftab), static_cast<const float4*>(tw));
  return hipGetLastError();
}

// complex filters: whole spectra, fp32 accumulation
template <class P, int NW, int CH, class TIO, bool CACHED>
static hipError_t launch_wave_complex(const void* u, const void* kf, void* y, int B, int H, const void* ftab,
                                      const void* tw, int, hipStream_t stream) {
  const unsigned grid = (unsigned)((H + CH - 1) / CH);
  hipLaunchKernelGGL((fftconv_wave_kernel<P, NW, CH, TIO, CACHED, false, false>), dim3(grid), dim3(64 * NW), 0,
                     stream, static_cast<const TIO*>(u), static_cast<const float4*>(kf), static_cast<TIO*>(y), B, H,
                     static_cast<const h8*>(ftab), static_cast<const float4*>(tw));
  return hipGetLastError();
}

template <int A, int B_, int C_, int W, int S>
static Entry make_entry() {
  typedef Plan<A, B_, C_> P;
  Entry e = {SFFFT_INST_L, A, B_, C_, W, S, 0, 1, P::LDS_BYTES,
             {{&launch_fused<P, W, S, float, false>, &launch_fused<P, W, S, float, true>},
              {&launch_fused<P, W, S, uint16_t, false>, &launch_fused<P, W, S, uint16_t, true>}},
             {{reinterpret_cast<const void*>(&fftconv_kernel<P, W, S, float, false, false, fused_wpe<P, W, false>()>),
               reinterpret_cast<const void*>(&fftconv_kernel<P, W, S, float, true, false, fused_wpe<P, W, true>()>)},
              {reinterpret_cast<const void*>(&fftconv_kernel<P, W, S, uint16_t, false, false, fused_wpe<P, W, false>()>),
               reinterpret_cast<const void*>(&fftconv_kernel<P, W, S, uint16_t, true, false, fused_wpe<P, W, true>()>)}},
             {{nullptr, nullptr}, {nullptr, nullptr}}};
  return e;
}

template <int A, int B_, int W, int CH>
static Entry make_wave_entry() {
  typedef WavePlan<A, B_> P;
  Entry e = {SFFFT_INST_L, A, B_, 1, W, 2, 1, CH, P::lds_bytes(CH, W),
             {{&launch_wave<P, W, CH, float, false>, &launch_wave<P, W, CH, float, true>},
              {&launch_wave<P, W, CH, uint16_t, false>, &launch_wave<P, W, CH, uint16_t, true>}},
             {{reinterpret_cast<const void*>(&fftconv_wave_kernel<P, W, CH, float, false, false, true>),
               reinterpret_cast<const void*>(&fftconv_wave_kernel<P, W, CH, float, true, false, true>)},
              {reinterpret_cast<const void*>(&fftconv_wave_kernel<P, W, CH, uint16_t, false, false, true>),
               reinterpret_cast<const void*>(&fftconv_wave_kernel<P, W, CH, uint16_t, true, false, true>)}},
             {{&launch_wave_complex<P, W, CH, float, false>, &launch_wave_complex<P, W, CH, float, true>},
              {&launch_wave_complex<P, W, CH, uint16_t, false>, &launch_wave_complex<P, W, CH, uint16_t, true>}}};
  return e;
}

#define SFFFT_PLAN(A, B_, C_, W) make_entry<A, B_, C_, W, 1>(), make_entry<A, B_, C_, W, 2>(),
#define SFFFT_WAVE(A, B_, W, CH) make_wave_entry<A, B_, W, CH>(),

static const Entry kEntries[] = {
#include "plans.def"
};

#define SFFFT_CAT_(a, b) a##b
#define SFFFT_CAT(a, b) SFFFT_CAT_(a, b)
const Entry* SFFFT_CAT(entries_L, SFFFT_INST_L)(int* n) {
  *n = (int)(sizeof(kEntries) / sizeof(kEntries[0]));
  return kEntries;
}

}  // namespace sffft
