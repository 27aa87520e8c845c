// Compiled-plan registry shared by the per-length instantiation units and the C ABI.
#pragma once
#include <hip/hip_runtime.h>

namespace sffft {

// Launches one instantiation. `tw` is the plan's twiddle table (wave pipeline only).
typedef hipError_t (*launch_fn)(const void* u, const void* kf, void* y, int B, int H, const void* ftab,
                                const void* tw, int acc16, hipStream_t stream);

// One (plan, waves, sequences-per-workgroup, mode) instantiation: launchers and kernel
// symbols for [io: 0 = fp32, 1 = bf16][cached: 0 = in-kernel DFT matrices, 1 = table].
//   mode 0: one workgroup per sequence (seqs = 1) or pair of sequences (seqs = 2),
//           stages exchanged through LDS (fftconv.hpp)
//   mode 1: one wavefront per pair of sequences, stages chained in VGPRs; a workgroup
//           of `waves` wavefronts takes `channels` channels and shares their spectra
//           and the DFT and twiddle tables in LDS (fftconv_wave.hpp; two-stage
//           plans, seqs = 2)
//   launch_complex: the same plan for complex filters (whole, non-Hermitian spectra
//           from sffft_spectrum_complex, fp32 accumulation); mode 1 only, else null
struct Entry {
  int L, r0, r1, r2, waves, seqs, mode, channels, lds_bytes;
  launch_fn launch[2][2];
  const void* func[2][2];
  launch_fn launch_complex[2][2];
};

// Defined by conv_inst.hip compiled once per length.
const Entry* entries_L128(int* n);
const Entry* entries_L256(int* n);
const Entry* entries_L512(int* n);
const Entry* entries_L1024(int* n);
const Entry* entries_L2048(int* n);
const Entry* entries_L4096(int* n);
const Entry* entries_L8192(int* n);
const Entry* entries_L16384(int* n);

// Multi-pass plans (mode 2, longconv.hpp): column radix nc, row plan r0 x r1; the three
// passes run on one stream with the caller's workspace.
// `chunk` channels per group of three launches (the workspace holds chunk*B/2 pairs).
typedef hipError_t (*long_launch_fn)(const void* u, const void* kf, void* y, void* work, int B, int H, int chunk,
                                     const void* ftab, const void* tw, hipStream_t stream);
struct LongEntry {
  int nc, r0, r1, lds_bytes;  // lds_bytes: the row pass's tables
  long_launch_fn launch[2][2];  // [0 = causal, 1 = circular of period 2L][io: 0 = fp32, 1 = bf16]
  const void* rows_func;      // the row-pass kernel (occupancy queries)
};
// Defined by long_inst.hip.
const LongEntry* long_entries(int* n);

}  // namespace sffft
