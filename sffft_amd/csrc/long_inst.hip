// Instantiates the multi-pass long-convolution kernels (longconv.hpp) and their
// launcher: pass A and pass C per (NC, I/O type), pass B per row plan (R0, R1); a
// compiled plan is any NC in {16, 32, 64} with any compiled row plan.
#include <mutex>

#include "longconv.hpp"
#include "registry.hpp"

namespace sffft {

// Workgroups of the row pass: as many as are resident on the device at once (the
// wavefronts loop over rows), so each workgroup copies the tables into LDS once.
template <int R0, int R1>
static unsigned rows_grid(int nrows) {
  static std::mutex mu;
  static int resident[256];  // per device: workgroups per CU * CUs (0 = not yet known)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 256) dev = 0;
  int n = 0;
  {
    std::lock_guard<std::mutex> lock(mu);
    if (!resident[dev]) {
      int per_cu = 0, cus = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(&long_rows<R0, R1>),
                                                       64 * LC_WAVES, 0) != hipSuccess ||
          per_cu < 1)
        per_cu = 1;
      if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
        cus = 256;
      resident[dev] = per_cu * cus;
    }
    n = resident[dev];
  }
  const int need = (nrows + LC_WAVES - 1) / LC_WAVES;
  return (unsigned)(need < n ? need : n);
}

// The three passes on one stream, for chunks of `chunk` channels: the workspace holds
// chunk*(B/2) pairs of N complex fp16 points. CIRC: circular convolution of period N.
template <int NC, int R0, int R1, class TIO, bool CIRC>
static hipError_t launch_long(const void* u, const void* kf, void* y, void* work, int B, int H, int chunk,
                              const void* ftab, const void* tw, hipStream_t s) {
  constexpr int NR = R0 * R1, N = NC * NR;
  const float inv_n = 1.0f / (float)N;  // exact: N is a power of two
  const int BP = B / 2;
  for (int h0 = 0; h0 < H; h0 += chunk) {
    const int nch = H - h0 < chunk ? H - h0 : chunk, pi0 = h0 * BP;
    const unsigned cgrid = (unsigned)((size_t)BP * nch * (NR / LC_CBLOCK));
    hipLaunchKernelGGL((long_cols_fwd<NC, TIO, CIRC>), dim3(cgrid), dim3(64 * LC_WAVES), 0, s,
                       static_cast<const TIO*>(u), static_cast<uint32_t*>(work), B, H, NR, pi0, inv_n,
                       static_cast<const h8*>(ftab));
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    const int nrows = nch * NC * BP;
    hipLaunchKernelGGL((long_rows<R0, R1>), dim3(rows_grid<R0, R1>(nrows)), dim3(64 * LC_WAVES), 0, s,
                       static_cast<uint32_t*>(work), static_cast<const float4*>(kf), nrows, BP, NC, h0, inv_n,
                       inv_sqrt_radix<NC>(), static_cast<const h8*>(ftab), static_cast<const float4*>(tw));
    if ((err = hipGetLastError()) != hipSuccess) return err;
    hipLaunchKernelGGL((long_cols_inv<NC, TIO, CIRC>), dim3(cgrid), dim3(64 * LC_WAVES), 0, s,
                       static_cast<const uint32_t*>(work), static_cast<TIO*>(y), B, H, NR, pi0,
                       static_cast<const h8*>(ftab));
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  return hipSuccess;
}

template <int NC, int R0, int R1>
static LongEntry make_long_entry() {
  LongEntry e = {NC, R0, R1, LongRowPlan<R0, R1>::LDS_BYTES,
                 {{&launch_long<NC, R0, R1, float, false>, &launch_long<NC, R0, R1, uint16_t, false>},
                  {&launch_long<NC, R0, R1, float, true>, &launch_long<NC, R0, R1, uint16_t, true>}},
                 reinterpret_cast<const void*>(&long_rows<R0, R1>)};
  return e;
}

#define SFFFT_LONG_ROWS(R0, R1) \
  make_long_entry<16, R0, R1>(), make_long_entry<32, R0, R1>(), make_long_entry<64, R0, R1>(),

static const LongEntry kLongEntries[] = {
    SFFFT_LONG_ROWS(16, 16) SFFFT_LONG_ROWS(32, 32) SFFFT_LONG_ROWS(64, 32) SFFFT_LONG_ROWS(64, 64)};

const LongEntry* long_entries(int* n) {
  *n = (int)(sizeof(kLongEntries) / sizeof(kLongEntries[0]));
  return kLongEntries;
}

}  // namespace sffft
