// Instantiates the fused kernel for every plan of one length (compiled once per
// length with -DSFFFT_INST_L=<L>, so the lengths build in parallel).
#include "fftconv.hpp"
#include "registry.hpp"

#ifndef SFFFT_INST_L
#error "compile with -DSFFFT_INST_L=<length>"
#endif

namespace sffft {

template <class P, int NW, int NSEQ, class TIO, bool CACHED>
static hipError_t launch_fused(const void* u, const void* kf, void* y, int B, int H, const void* ftab, int acc16,
                               hipStream_t stream) {
  const unsigned grid = (unsigned)(H * (B / NSEQ));
  hipLaunchKernelGGL((fftconv_kernel<P, NW, NSEQ, TIO, CACHED>), dim3(grid), dim3(64 * NW), 0, stream,
                     static_cast<const TIO*>(u), static_cast<const float2*>(kf), static_cast<TIO*>(y), B, H,
                     static_cast<const h8*>(ftab), acc16);
  return hipGetLastError();
}

template <class P, int NW, int NSEQ, class TIO, bool CACHED>
static const void* kernel_symbol() {
  return reinterpret_cast<const void*>(&fftconv_kernel<P, NW, NSEQ, TIO, CACHED>);
}

template <int A, int B_, int C_, int W, int S>
static Entry make_entry() {
  typedef Plan<A, B_, C_> P;
  Entry e = {SFFFT_INST_L, A, B_, C_, W, S, P::LDS_BYTES,
             {{&launch_fused<P, W, S, float, false>, &launch_fused<P, W, S, float, true>},
              {&launch_fused<P, W, S, uint16_t, false>, &launch_fused<P, W, S, uint16_t, true>}},
             {{kernel_symbol<P, W, S, float, false>(), kernel_symbol<P, W, S, float, true>()},
              {kernel_symbol<P, W, S, uint16_t, false>(), kernel_symbol<P, W, S, uint16_t, true>()}}};
  return e;
}

#define SFFFT_PLAN(A, B_, C_, W) make_entry<A, B_, C_, W, 1>(), make_entry<A, B_, C_, W, 2>(),

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
