// C ABI of libsffft.so: plan checks, the DFT coefficient table, filter-spectrum
// preparation, the fused convolution launch and the host-side selector.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstring>
#include <limits>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "../../include/sffft.h"
#include "fftconv.hpp"
#include "fftconv_wave.hpp"
#include "longconv.hpp"
#include "registry.hpp"
#include "transforms.hpp"

// Workspace of sffft_spectrum_noalloc, the one entry point that allocates nothing: a
// static device array, one per GPU the library runs on, held until the process ends.
// Host code never uses its name as an address (that is a host-side stand-in): the device
// address comes from hipGetSymbolAddress, once per device (scratch_for_device).
static constexpr size_t SFFFT_SCRATCH_BYTES = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[SFFFT_SCRATCH_BYTES];

namespace sffft {
namespace {

thread_local char g_last_error[256] = "";

// Records the HIP error of the last failing call on this thread.
int hip_status(hipError_t err, const char* what) {
  if (err == hipSuccess) return SFFFT_OK;
  snprintf(g_last_error, sizeof(g_last_error), "%s: %s (%d)", what, hipGetErrorString(err), (int)err);
  return SFFFT_EHIP;
}

bool valid_radix(int r) { return r == 16 || r == 32 || r == 64; }
// single-pass plans (modes 0 and 1) up to L = 16384; multi-pass plans (mode 2) up to
// L = 131072 (N = 64 * 64 * 64)
constexpr int MAX_SINGLE_L = 16384, MAX_LONG_L = 131072;
bool valid_length(int L) { return L >= 128 && L <= MAX_LONG_L && (L & (L - 1)) == 0; }
// mode 0: 1, 2, 4, 8 or 16 wavefronts; mode 1 (one pair per wavefront): 1..16;
// mode 2: the four wavefronts of every pass
bool valid_waves(int w, int mode) {
  if (mode == 2) return w == LC_WAVES;
  return mode == 1 ? (w >= 1 && w <= 16) : (w == 1 || w == 2 || w == 4 || w == 8 || w == 16);
}

// Same formulas as Plan<>::LDS_BYTES and WavePlan<>::LDS_BYTES, for plans that are
// not compiled.
size_t lds_bytes_rt(int r0, int r1, int r2, int mode, int channels, int waves) {
  if (mode == 2) {
    // LongRowPlan::LDS_BYTES of the row plan r1 x r2: first-kind DFT fragments and the
    // twiddle table(s)
    const int T1 = r1 / 16, T2 = r2 / 16, NR = r1 * r2;
    return (size_t)(T1 * T1 * 64 + (r2 == r1 ? 0 : T2 * T2 * 64)) * 16 + (size_t)(r2 == r1 ? 1 : 2) * NR * 8;
  }
  if (mode == 1) {
    // WavePlan::lds_bytes: the twiddle tables (one when r0 == r1), the row-load scratch and,
    // in order of preference, both DFT fragment kinds and the spectra; the first kind only
    // and the spectra; or the first kind only (spectra read through L2). The spectra are
    // Hermitian halves (WavePlan::HSP_F4 float4 per channel) in whole 64-float4 runs.
    const int T0 = r0 / 16, T1 = r1 / 16, N = r0 * r1;
    const size_t frags = (size_t)(T0 * T0 * 128 + (r1 == r0 ? 0 : T1 * T1 * 128)) * 16;
    const size_t tw = (size_t)((r1 == r0 ? 1 : 2) * N / 2) * 16;
    const size_t half_f4 = (size_t)(r0 / 2 + 1) * (8 * T1 + 1);
    const size_t scratch = (size_t)waves * 16 * (r1 + 4) * 4, spectra = (channels * half_f4 + 63) / 64 * 64 * 16;
    const size_t tab = frags + tw + spectra + scratch <= 163840 ? frags + tw : frags / 2 + tw;
    const bool in_lds = tab + spectra + scratch <= 163840;
    return tab + (in_lds ? spectra : 0) + scratch;
  }
  const int S = r2 > 1 ? 3 : 2, N = r0 * r1 * r2, M = N / r0;
  const int PA = r1 + LDS_PAD, PB = r0 + LDS_PAD;
  const int ROW = S == 3 ? r2 * PA : 0;
  const int P0 = S == 3 ? r0 * ROW : cmax(r0 * PA, r1 * PB);
  return (size_t)(((P0 + 63) & ~63) * 4);
}

const Entry* entries_for(int L, int* n) {
  switch (L) {
    case 128: return entries_L128(n);
    case 256: return entries_L256(n);
    case 512: return entries_L512(n);
    case 1024: return entries_L1024(n);
    case 2048: return entries_L2048(n);
    case 4096: return entries_L4096(n);
    case 8192: return entries_L8192(n);
    case 16384: return entries_L16384(n);
    default: *n = 0; return nullptr;
  }
}

int check_shape(int L, const sffft_plan* p) {
  if (!p || !valid_length(L)) return SFFFT_EINVAL;
  if (p->mode != 2 && L > MAX_SINGLE_L) return SFFFT_EINVAL;
  if (!valid_radix(p->r0) || !valid_radix(p->r1) || !(p->r2 == 1 || valid_radix(p->r2))) return SFFFT_EINVAL;
  if ((long long)p->r0 * p->r1 * p->r2 != 2LL * L) return SFFFT_EINVAL;
  if (!valid_waves(p->waves, p->mode) || (p->acc != 0 && p->acc != 1) || (p->cached != 0 && p->cached != 1) ||
      (p->seqs != 1 && p->seqs != 2) || p->mode < 0 || p->mode > 2 || p->channels < 1 || p->channels > 16)
    return SFFFT_EINVAL;
  // multi-pass: three radices (column radix r0, row plan r1 x r2), pairs of sequences,
  // fp32 accumulation, DFT fragments from the coefficient table
  if (p->mode == 2 && (p->r2 == 1 || p->seqs != 2 || p->channels != 1 || p->acc != 0 || p->cached != 1))
    return SFFFT_EINVAL;
  if (p->mode == 0 && p->channels != 1) return SFFFT_EINVAL;
  if (p->mode == 1 && (p->r2 != 1 || p->seqs != 2)) return SFFFT_EINVAL;
  if (p->mode == 0 && p->r2 > 1 && p->r0 % p->waves) return SFFFT_EINVAL;
  if (lds_bytes_rt(p->r0, p->r1, p->r2, p->mode, p->channels, p->waves) > 163840) return SFFFT_EINVAL;
  return SFFFT_OK;
}

const LongEntry* find_long_entry(const sffft_plan* p) {
  if (p->mode != 2) return nullptr;
  int n = 0;
  const LongEntry* e = long_entries(&n);
  for (int i = 0; i < n; i++)
    if (e[i].nc == p->r0 && e[i].r0 == p->r1 && e[i].r1 == p->r2) return &e[i];
  return nullptr;
}

const Entry* find_entry(int L, const sffft_plan* p) {
  if (p->mode == 2) return nullptr;
  int n = 0;
  const Entry* e = entries_for(L, &n);
  for (int i = 0; i < n; i++)
    if (e[i].r0 == p->r0 && e[i].r1 == p->r1 && e[i].r2 == p->r2 && e[i].waves == p->waves &&
        e[i].seqs == p->seqs && e[i].mode == p->mode && e[i].channels == p->channels)
      return &e[i];
  return nullptr;
}

// ---- DFT coefficient table (the "cached" DFT matrices, src/sffft.cu:349-362) ----
// Entries are __float2half((float)cos(angle)) / (float)-sin(angle) of the exact
// angle 2*pi*(e mod R)/R, as in the reference table, arranged as MFMA fragments.
void build_table(std::vector<_Float16>& t) {
  t.assign((size_t)FTAB_H8 * 8, (_Float16)0.f);
  const double two_pi = 6.283185307179586476925286766559;
  auto cs = [&](int e, int R, float* c, float* s) {
    const double a = two_pi * (double)(e % R) / (double)R;
    *c = (float)std::cos(a);
    *s = (float)std::sin(a);
  };
  for (int R : {16, 32, 64}) {
    const int T = R / 16;
    for (int a = 0; a < T; a++)
      for (int b = 0; b < T; b++)
        for (int kind = 0; kind < 2; kind++)
          for (int lane = 0; lane < 64; lane++) {
            const int r = lane & 15, g = lane >> 4;
            _Float16* f = &t[((size_t)cf_off(R) + ((a * T + b) * 2 + kind) * 64 + lane) * 8];
            for (int v = 0; v < 4; v++) {
              float c, s;
              cs((16 * a + r) * (16 * b + 4 * g + v), R, &c, &s);
              f[v] = (_Float16)(kind == 0 ? c : -s);
              f[4 + v] = (_Float16)(kind == 0 ? s : c);
            }
          }
    for (int nt = 0; nt < T; nt++)
      for (int kind = 0; kind < 2; kind++)
        for (int lane = 0; lane < 64; lane++) {
          const int c16 = lane & 15, g = lane >> 4;
          _Float16* f = &t[((size_t)ri_off(R) + (nt * 2 + kind) * 64 + lane) * 8];
          for (int j = 0; j < 8; j++) {
            const int n0 = j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4);
            float c, s;
            cs(n0 * (16 * nt + c16), R, &c, &s);
            f[j] = n0 >= R / 2 ? (_Float16)0.f : (_Float16)(kind == 0 ? c : -s);
          }
        }
  }
}

std::mutex g_table_mu;
void* g_table[256];

int device_table(const void** out) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return hip_status(err, "hipGetDevice");
  if (dev < 0 || dev >= 256) return SFFFT_EINVAL;
  std::lock_guard<std::mutex> lock(g_table_mu);
  if (!g_table[dev]) {
    std::vector<_Float16> host;
    build_table(host);
    void* d = nullptr;
    if ((err = hipMalloc(&d, host.size() * sizeof(_Float16))) != hipSuccess) return hip_status(err, "hipMalloc");
    if ((err = hipMemcpy(d, host.data(), host.size() * sizeof(_Float16), hipMemcpyHostToDevice)) != hipSuccess) {
      (void)hipFree(d);
      return hip_status(err, "hipMemcpy");
    }
    g_table[dev] = d;
  }
  *out = g_table[dev];
  return SFFFT_OK;
}

// ---- twiddle tables of the wave pipeline (fftconv_wave.hpp) ---------------------
// TW1[tile mt*ST+nt][lane (c,g)][v] = sc0 * w^(m k0),        m = 16mt+4g+v, k0 = 16nt+c
// TW2[tile s*MT+t][lane (c,g)][v]   = sc0 * sc1 * w^(k0 n1), k0 = 16s+4g+v,  n1 = 16t+c
// (complex fp32, at float4 tw_index(split, tile, lane, v / 2), slot v % 2: the wave pipeline's
// layout is tw_split(r0, r1), the multi-pass row pass's the paired one)
// with w = exp(-2 pi i / N), sc = 1/sqrt(R); exponents reduced mod N, fp64 then fp32.
// Square plans (r0 == r1) read TW1 only: TW2 equals it index for index up to sc1,
// which their spectrum carries instead (last_stage_scale).
void build_twiddles(int r0, int r1, bool split, std::vector<float>& t) {
  const int N = r0 * r1, ST = r0 / 16, MT = r1 / 16;
  const double two_pi = 6.283185307179586476925286766559;
  const double sc0 = 1.0 / std::sqrt((double)r0), sc1 = 1.0 / std::sqrt((double)r1);
  t.assign((size_t)2 * N * 2, 0.f);
  auto put = [&](size_t base, int tile, int lane, int v, long long e, double sc) {
    e %= N;
    if (e > N / 2) e -= N;
    const double a = two_pi * (double)e / (double)N;
    float* f = &t[base + (size_t)tw_index(split, tile, lane, v / 2) * 4 + 2 * (v % 2)];
    f[0] = (float)(sc * std::cos(a));
    f[1] = (float)(-sc * std::sin(a));
  };
  for (int mt = 0; mt < MT; mt++)
    for (int nt = 0; nt < ST; nt++)
      for (int lane = 0; lane < 64; lane++)
        for (int v = 0; v < 4; v++) {
          const int c = lane & 15, g = lane >> 4;
          put(0, mt * ST + nt, lane, v, (long long)(16 * mt + 4 * g + v) * (16 * nt + c), sc0);
        }
  for (int s = 0; s < ST; s++)
    for (int tt = 0; tt < MT; tt++)
      for (int lane = 0; lane < 64; lane++)
        for (int v = 0; v < 4; v++) {
          const int c = lane & 15, g = lane >> 4;
          put((size_t)2 * N, s * MT + tt, lane, v, (long long)(16 * s + 4 * g + v) * (16 * tt + c), sc0 * sc1);
        }
}

// Layout 2 (the fp16-products kernels): the same values rounded to fp16, one 16-byte entry
// per (tile, lane) at h8 index tile * 64 + lane, [wr0 wr1 wr2 wr3 | wi0 wi1 wi2 wi3]; TW2
// after TW1's N complex values.
void build_twiddles_h(int r0, int r1, std::vector<_Float16>& t) {
  const int N = r0 * r1;
  std::vector<float> f;
  build_twiddles(r0, r1, true, f);  // split layout: value v of (tile, lane) at float4 (tile*2 + v/2)*64 + lane
  t.assign((size_t)2 * N * 2, (_Float16)0.f);
  const int tiles = N / 256;
  for (int part = 0; part < 2; part++)
    for (int tile = 0; tile < tiles; tile++)
      for (int lane = 0; lane < 64; lane++)
        for (int v = 0; v < 4; v++) {
          const float* src = &f[(size_t)part * 2 * N + (size_t)tw_index(true, tile, lane, v / 2) * 4 + 2 * (v % 2)];
          _Float16* dst = &t[(size_t)part * 2 * N + ((size_t)tile * 64 + lane) * 8];
          dst[v] = (_Float16)src[0];
          dst[4 + v] = (_Float16)src[1];
        }
}

std::mutex g_scratch_mu;
void* g_scratch[256];  // per device: the device address of `scratch`

// The current device's copy of `scratch`, looked up on the first call on that device.
int scratch_for_device(void** out) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return hip_status(err, "hipGetDevice");
  if (dev < 0 || dev >= 256) return SFFFT_EINVAL;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    if ((err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) != hipSuccess)
      return hip_status(err, "hipGetSymbolAddress(scratch)");
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return SFFFT_OK;
}

std::mutex g_tw_mu;
std::map<std::tuple<int, int, int>, void*> g_tw[256];  // per device: (r0, r1, layout) -> table

// Twiddle tables of plan r0 x r1 in `layout`: 0 paired (fp32), 1 split (fp32), 2 fp16.
int device_twiddles(int r0, int r1, int layout, const void** out) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return hip_status(err, "hipGetDevice");
  if (dev < 0 || dev >= 256) return SFFFT_EINVAL;
  std::lock_guard<std::mutex> lock(g_tw_mu);
  void*& slot = g_tw[dev][std::make_tuple(r0, r1, layout)];
  if (!slot) {
    std::vector<float> host32;
    std::vector<_Float16> host16;
    if (layout == 2)
      build_twiddles_h(r0, r1, host16);
    else
      build_twiddles(r0, r1, layout == 1, host32);
    const void* src = layout == 2 ? (const void*)host16.data() : (const void*)host32.data();
    const size_t bytes = layout == 2 ? host16.size() * sizeof(_Float16) : host32.size() * sizeof(float);
    void* d = nullptr;
    if ((err = hipMalloc(&d, bytes)) != hipSuccess) return hip_status(err, "hipMalloc");
    if ((err = hipMemcpy(d, src, bytes, hipMemcpyHostToDevice)) != hipSuccess) {
      (void)hipFree(d);
      return hip_status(err, "hipMemcpy");
    }
    slot = d;
  }
  *out = slot;
  return SFFFT_OK;
}

// ---- filter spectrum ----------------------------------------------------------
// Runtime form of kernel_order_digits<P> (mode 0) and of the wave pipeline's order
// sp_index (mode 1: complex idx = 2*sp_index(s*MT + kt, lane, q) + e holds value
// v = 2q + e of lane (c, g): k0 = 16s + c, k1 = 16kt + 4g + v).
__device__ inline void kernel_order_digits_rt(int idx, int r0, int r1, int r2, int mode, int& k0, int& k1,
                                              int& k2) {
  if (mode == 1) {
    const int e = idx & 1, lane = (idx >> 1) & 63, rest = idx >> 7;
    const int q = rest & 1, tile = rest >> 1, MT = r1 / 16;
    const int c = lane & 15, g = lane >> 4;
    k0 = 16 * (tile / MT) + c;
    k1 = 16 * (tile % MT) + 4 * g + 2 * q + e;
    k2 = 0;
    return;
  }
  const int v = idx & 3, lane = (idx >> 2) & 63, rest = idx >> 8;
  const int c = lane & 15, g = lane >> 4;
  if (r2 == 1) {
    const int T1 = r1 / 16, mt = rest % T1, s = rest / T1;
    k0 = 16 * s + c;
    k1 = 16 * mt + 4 * g + v;
    k2 = 0;
  } else {
    const int T1 = r1 / 16, T2 = r2 / 16;
    const int mt = rest % T2, t1 = (rest / T2) % T1;
    k0 = rest / (T2 * T1);
    k1 = 16 * t1 + c;
    k2 = 16 * mt + 4 * g + v;
  }
}

// Gather of a natural-order spectrum into the fused kernel's order, folding in
// 1/sqrt(R_last) of the last forward stage: real parts times scale, imaginary parts times
// iscale (-scale gathers the conjugate spectrum).
__global__ void spectrum_permute_kernel(const float2* __restrict__ src, float2* __restrict__ kf, int H, int r0,
                                        int r1, int r2, int mode, float scale, float iscale) {
  const int N = r0 * r1 * r2;
  const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (size_t)H * N) return;
  const int h = (int)(gid / N), idx = (int)(gid % N);
  int k0, k1, k2, s;
  if (mode == 2) {
    // multi-pass: row k1 = idx / NR holds the row plan's spectrum order (the wave
    // pipeline's sp_index over the row plan r1 x r2) of frequencies k1 + r0*(k0' + r1*k1')
    const int NR = r1 * r2, row = idx / NR;
    kernel_order_digits_rt(idx - row * NR, r1, r2, 1, 1, k0, k1, k2);
    s = row + r0 * (k0 + r1 * k1);
  } else {
    kernel_order_digits_rt(idx, r0, r1, r2, mode, k0, k1, k2);
    s = k0 + r0 * k1 + r0 * r1 * k2;
  }
  const float2 v = src[(size_t)h * N + s];
  kf[gid] = make_float2(v.x * scale, v.y * iscale);
}

// Hermitian half of a real filter's spectrum in the wave pipeline's order
// (WavePlan::hs_index): per channel, (r0/2 + 1) columns k0 of PITCH = 8*(r1/16) + 1
// float4; float4 (k0*PITCH + (kt*2 + q)*4 + g) holds k1 = 16kt + 4g + 2q and +1, i.e.
// K[k0 + r0*k1]. Column r0/2 holds conj(K[r0/2 + r0*(r1 - 1 - k1)]) at k1; the last float4
// of each column is zero padding. src as in spectrum_permute_kernel, for the H channels
// from channel h0 on. Each channel keeps its own row of the [H][N] complex64 buffer: its
// C = 2*(r0/2 + 1)*PITCH values first, zeros after them, so a row of kf is a channel for
// every plan (slices and concatenations of spectra along the channels stay valid).
__global__ void spectrum_half_kernel(const float2* __restrict__ src, float2* __restrict__ kf, int H, int h0, int r0,
                                     int r1, float scale, float iscale) {
  const int pitch = 8 * (r1 / 16) + 1, C = 2 * (r0 / 2 + 1) * pitch, N = r0 * r1;
  const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (size_t)H * N) return;
  float2* out = kf + (size_t)h0 * N + gid;
  const int h = (int)(gid / N), i = (int)(gid % N);
  const int f = i >> 1, e = i & 1, k0 = f / pitch, rem = f % pitch;
  if (i >= C || rem == pitch - 1) {
    *out = make_float2(0.f, 0.f);
    return;
  }
  const int g = rem & 3, q = (rem >> 2) & 1, kt = rem >> 3;
  const int k1 = 16 * kt + 4 * g + 2 * q + e;
  const bool mid = k0 == r0 / 2;
  const int kk1 = mid ? r1 - 1 - k1 : k1;
  const int sidx = k0 + r0 * kk1;
  const float2 v = src[(size_t)h * N + sidx];
  *out = make_float2(v.x * scale, (mid ? -v.y : v.y) * iscale);
}

// Filter rows kr[h][0..klen) (+ i ki[h][..] for a complex filter, ki may be null) as complex
// rows of length N, zero-padded: the spectrum's input.
__global__ void spectrum_pad_kernel(const float* __restrict__ kr, const float* __restrict__ ki,
                                    float2* __restrict__ w, int klen, int N, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const size_t h = i / (size_t)N;
  const int p = (int)(i - h * (size_t)N);
  const size_t j = h * (size_t)klen + p;
  w[i] = p < klen ? make_float2(kr[j], ki ? ki[j] : 0.f) : make_float2(0.f, 0.f);
}

__global__ void to_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ y, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = f32_to_bf16(x[i]);
}

// Scale folded into the kernel-order spectrum: 1/sqrt(R) of the last radix; square
// wave plans also carry the 1/sqrt(R1) of their shared twiddle table (1/R1 in all).
float last_stage_scale(const sffft_plan* p) {
  const int R = p->r2 > 1 ? p->r2 : p->r1;
  // multi-pass: the row plan r1 x r2's factor (its forward DFT over n1 of radix r2)
  if (p->mode == 2) return (float)(p->r1 == p->r2 ? 1.0 / (double)R : 1.0 / std::sqrt((double)R));
  if (p->mode == 1 && p->r0 == p->r1) return (float)(1.0 / (double)R);
  return (float)(1.0 / std::sqrt((double)R));
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Test probe of the in-register twiddles of the workgroup kernel (fftconv.hpp): query q =
// (e0, step, f0, fstep) gives the four values twiddle4e<N>(e0, step, sc) and `rows` row
// steps, each the complex product with twiddle4e<N>(f0, fstep, 1) (the row recurrence of the
// kernel's phase-2 loop), stored as out[q][row][v] complex64, row = 0..rows.
template <int N>
__global__ void twiddle_probe_kernel(const int4* __restrict__ qs, float2* __restrict__ out, int nq, int rows,
                                     float sc) {
  const int q = blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= nq) return;
  const int4 a = qs[q];
  float wr[4], wi[4], fr[4], fi[4];
  twiddle4e<N>(a.x, a.y, sc, wr, wi);
  twiddle4e<N>(a.z, a.w, 1.f, fr, fi);
  float2* o = out + (size_t)q * (rows + 1) * 4;
  for (int r = 0;; r++) {
#pragma unroll
    for (int v = 0; v < 4; v++) o[r * 4 + v] = make_float2(wr[v], wi[v]);
    if (r == rows) break;
    cmul4(wr, wi, fr, fi);
  }
}

// Body-less kernel: launched with a plan's grid, block and LDS size it measures the
// dispatch cost of that launch shape (workgroup dispatch, LDS allocation, wave
// launch and retirement) without any memory traffic.
__global__ void empty_dispatch_kernel() {}

// cplx: complex filters (whole spectra from sffft_spectrum_complex); wave plans then run
// their non-Hermitian instantiation, the other plans read whole spectra anyway.
template <int IO>
int conv(const void* u, const void* kf, void* y, int B, int H, int L, const sffft_plan* p, void* stream,
         int cplx = 0) {
  if (!u || !kf || !y || B < 1 || H < 1 || (long long)B * H > INT_MAX) return SFFFT_EINVAL;
  int rc = check_shape(L, p);
  if (rc) return rc;
  if (B % p->seqs) return SFFFT_EINVAL;
  if (p->mode == 2) return SFFFT_EINVAL;  // multi-pass plans need a workspace: sffft_conv_long_*
  if (!aligned16(u) || !aligned16(y) || !aligned16(kf)) return SFFFT_EINVAL;
  const Entry* e = find_entry(L, p);
  if (!e) return SFFFT_ENOPLAN;
  const void* table = nullptr;
  if ((rc = device_table(&table))) return rc;
  const void* tw = nullptr;
  // wave plans: the fp16 tables for the fp16-products kernels (the fp16-accumulation
  // mode, real filters), else the fp32 tables in the plan's layout
  const bool hp = e->mode == 1 && !cplx && p->acc;
  if (e->mode == 1 && (rc = device_twiddles(p->r0, p->r1, hp ? 2 : tw_split(p->r0, p->r1) ? 1 : 0, &tw))) return rc;
  const launch_fn fn = cplx && e->mode == 1 ? e->launch_complex[IO][p->cached] : e->launch[IO][p->cached];
  return hip_status(fn(u, kf, y, B, H, table, tw, p->acc, (hipStream_t)stream), "fused convolution launch");
}

// Workspace of one channel (its B/2 pairs of 2L complex fp16 points); a workspace of
// c channels runs the batch in ceil(H/c) chunks.
size_t channel_work_bytes(int B, int L) { return (size_t)(B / 2) * 2 * L * 4; }
// Default workspace: chunks of at most 96 MiB (kept in the 256 MB Infinity Cache
// between the passes), or the whole batch when it is smaller.
size_t work_bytes(int B, int H, int L) {
  const size_t per = channel_work_bytes(B, L), cap = (size_t)96 << 20;
  size_t ch = cap / per;
  if (ch < 1) ch = 1;
  if (ch > (size_t)H) ch = (size_t)H;
  return ch * per;
}

// circ: circular convolution of period 2L (rows of length 2L)
template <int IO>
int conv_long(const void* u, const void* kf, void* y, void* work, size_t wbytes, int B, int H, int L,
              const sffft_plan* p, void* stream, int circ = 0) {
  if (!u || !kf || !y || !work || B < 2 || H < 1 || (long long)B * H > INT_MAX) return SFFFT_EINVAL;
  int rc = check_shape(L, p);
  if (rc) return rc;
  if (p->mode != 2 || B % 2) return SFFFT_EINVAL;
  if (!aligned16(u) || !aligned16(y) || !aligned16(kf) || !aligned16(work)) return SFFFT_EINVAL;
  if (wbytes < channel_work_bytes(B, L)) return SFFFT_EINVAL;
  const size_t chunk_sz = wbytes / channel_work_bytes(B, L);
  const int chunk = chunk_sz < (size_t)H ? (int)chunk_sz : H;
  // row counts of the passes are int
  if ((long long)H * p->r0 * (B / 2) > INT_MAX || (long long)(B / 2) * H * (p->r1 * p->r2 / LC_CBLOCK) > INT_MAX)
    return SFFFT_EINVAL;
  // the workspace must not overlap the input, output or spectrum
  auto overlaps = [](const void* a, size_t na, const void* b, size_t nb) {
    const uintptr_t x = (uintptr_t)a, z = (uintptr_t)b;
    return x < z + nb && z < x + na;
  };
  const size_t io_bytes = (size_t)B * H * L * (circ ? 2 : 1) * (IO ? 2 : 4);
  wbytes = (size_t)chunk * channel_work_bytes(B, L);  // the part the passes use
  if (overlaps(work, wbytes, u, io_bytes) || overlaps(work, wbytes, y, io_bytes) ||
      overlaps(work, wbytes, kf, (size_t)H * 2 * L * 8))
    return SFFFT_EINVAL;
  const LongEntry* e = find_long_entry(p);
  if (!e) return SFFFT_ENOPLAN;
  const void* table = nullptr;
  if ((rc = device_table(&table))) return rc;
  const void* tw = nullptr;
  if ((rc = device_twiddles(p->r1, p->r2, 0, &tw))) return rc;
  return hip_status(e->launch[circ][IO](u, kf, y, work, B, H, chunk, table, tw, (hipStream_t)stream),
                    "multi-pass launch");
}

// Compiled multi-pass plans of length L, in registry order.
int long_plans_for(int L, const LongEntry** out, int cap) {
  int n = 0, k = 0;
  const LongEntry* e = long_entries(&n);
  for (int i = 0; i < n; i++)
    if ((long long)e[i].nc * e[i].r0 * e[i].r1 == 2LL * L) {
      if (k < cap) out[k] = &e[i];
      k++;
    }
  return k;
}

// Launches the gather of a natural-order spectrum src of the H channels from channel h0 on
// into the kernel order of the plan: the Hermitian half for wave plans (mode 1) unless
// `whole` (complex filters), else the whole spectrum; with conj, of the conjugate spectrum.
// Channel h is row h of kf ([H][N] complex64) in every case.
int permute_launch(const float2* src, float2* kf, int H, const sffft_plan* plan, int whole, int conj, hipStream_t s,
                   int h0 = 0) {
  const float sc = last_stage_scale(plan), isc = conj ? -sc : sc;
  const size_t N = (size_t)plan->r0 * plan->r1 * plan->r2, total = (size_t)H * N;
  if (plan->mode == 1 && !whole)
    hipLaunchKernelGGL(spectrum_half_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, src, kf, H, h0,
                       plan->r0, plan->r1, sc, isc);
  else
    hipLaunchKernelGGL(spectrum_permute_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, src,
                       kf + (size_t)h0 * N, H, plan->r0, plan->r1, plan->r2, plan->mode, sc, isc);
  return hip_status(hipGetLastError(), "spectrum permute launch");
}

// Spectrum of the H filter rows from channel h0 on: kr, plus
// i ki for a complex filter (ki non-null, whole spectrum); with conj, its conjugate (the
// spectrum the correlations of the backward passes run on). The padded rows are transformed
// in place in `work` (H * N complex64; fp64 stages, complex64 between them), then gathered
// into kernel order. Up to 16384 points the transform is one pass through LDS and needs no
// workspace. Longer rows take the two-pass transform, whose workspace is this call's own rows
// of kf: the gather overwrites them afterwards, and the results of earlier calls (the rows
// of the channels before h0) lie before them.
int spectrum_impl(const float* kr, const float* ki, int H, int L, int klen, const sffft_plan* plan, void* kf,
                  void* work, void* stream, int whole = 0, int conj = 0, int h0 = 0) {
  if (!kr || !kf || !work || H < 1 || kf == work) return SFFFT_EINVAL;
  const int rc = check_shape(L, plan);
  if (rc) return rc;
  const int N = 2 * L;
  hipStream_t s = (hipStream_t)stream;
  float2* w = static_cast<float2*>(work);
  const size_t off = (size_t)h0 * klen, n = (size_t)H * N;
  hipLaunchKernelGGL(spectrum_pad_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, kr + off,
                     ki ? ki + off : nullptr, w, klen, N, n);
  int st = hip_status(hipGetLastError(), "spectrum pad launch");
  if (st) return st;
  const xf::Seqs q{H, 1, 0, N, 1, 0};
  float2* scratch = N <= xf::ONEPASS_MAX_N ? nullptr : static_cast<float2*>(kf) + (size_t)h0 * N;
  if ((st = hip_status(xf::run(w, w, scratch, q, N, 0, 1.f, s), "spectrum transform launch"))) return st;
  return permute_launch(w, static_cast<float2*>(kf), H, plan, whole, conj, s, h0);
}
}  // namespace
}  // namespace sffft

using namespace sffft;

extern "C" {

int sffft_plan_check(int L, const sffft_plan* plan) {
  const int rc = check_shape(L, plan);
  if (rc) return rc;
  if (plan->mode == 2) return find_long_entry(plan) ? SFFFT_OK : SFFFT_ENOPLAN;
  return find_entry(L, plan) ? SFFFT_OK : SFFFT_ENOPLAN;
}

size_t sffft_plan_lds_bytes(int L, const sffft_plan* plan) {
  if (check_shape(L, plan)) return 0;
  return lds_bytes_rt(plan->r0, plan->r1, plan->r2, plan->mode, plan->channels, plan->waves);
}

int sffft_plan_occupancy(int L, const sffft_plan* plan, int* blocks_per_cu) {
  if (!blocks_per_cu) return SFFFT_EINVAL;
  const int rc = sffft_plan_check(L, plan);
  if (rc) return rc;
  const Entry* e = find_entry(L, plan);
  const void* func = plan->mode == 2 ? find_long_entry(plan)->rows_func : e->func[0][plan->cached];
  int n = 0;
  const int st = hip_status(
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, func, 64 * plan->waves, 0),
      "hipOccupancyMaxActiveBlocksPerMultiprocessor");
  if (st) return st;
  *blocks_per_cu = n;
  return SFFFT_OK;
}

int sffft_plan_count(int L) {
  if (L > MAX_SINGLE_L) return valid_length(L) ? long_plans_for(L, nullptr, 0) : 0;
  int n = 0;
  entries_for(L, &n);
  return n;
}

int sffft_plan_get(int L, int index, sffft_plan* plan, char* name, size_t name_len) {
  if (L > MAX_SINGLE_L) {
    const LongEntry* le[64];
    const int n = valid_length(L) ? long_plans_for(L, le, 64) : 0;
    if (index < 0 || index >= n || index >= 64) return SFFFT_ENOTFOUND;
    if (plan) *plan = sffft_plan{le[index]->nc, le[index]->r0, le[index]->r1, LC_WAVES, 0, 1, 2, 2, 1};
    if (name && name_len) snprintf(name, name_len, "%dx%dx%d", le[index]->nc, le[index]->r0, le[index]->r1);
    return SFFFT_OK;
  }
  int n = 0;
  const Entry* e = entries_for(L, &n);
  if (index < 0 || index >= n) return SFFFT_ENOTFOUND;
  if (plan) {
    plan->r0 = e[index].r0;
    plan->r1 = e[index].r1;
    plan->r2 = e[index].r2;
    plan->waves = e[index].waves;
    plan->seqs = e[index].seqs;
    plan->mode = e[index].mode;
    plan->channels = e[index].channels;
    plan->acc = 0;
    plan->cached = 1;
  }
  if (name && name_len) {
    if (e[index].r2 > 1)
      snprintf(name, name_len, "%dx%dx%d", e[index].r0, e[index].r1, e[index].r2);
    else
      snprintf(name, name_len, "%dx%d", e[index].r0, e[index].r1);
  }
  return SFFFT_OK;
}

size_t sffft_spectrum_bytes(int H, int L) {
  if (H < 1 || !valid_length(L)) return 0;
  return (size_t)H * 2 * L * 8;
}

int sffft_spectrum(const float* k, int H, int L, const sffft_plan* plan, void* kf, void* work, void* stream) {
  return spectrum_impl(k, nullptr, H, L, L, plan, kf, work, stream);
}

int sffft_spectrum_conj(const float* k, int H, int L, const sffft_plan* plan, void* kf, void* work, void* stream) {
  return spectrum_impl(k, nullptr, H, L, L, plan, kf, work, stream, 0, 1);
}

int sffft_spectrum_noalloc(const float* k, int H, int L, const sffft_plan* plan, void* kf, void* stream) {
  if (!k || !kf || H < 1) return SFFFT_EINVAL;
  int rc = check_shape(L, plan);
  if (rc) return rc;
  const size_t per = (size_t)2 * L * 8;  // one channel staged through the workspace
  if (per > SFFFT_SCRATCH_BYTES) {
    snprintf(g_last_error, sizeof(g_last_error), "sffft_spectrum_noalloc: one channel needs %zu bytes of "
             "workspace, the static scratch holds %zu", per, SFFFT_SCRATCH_BYTES);
    return SFFFT_ESCRATCH;
  }
  void* work = nullptr;
  if ((rc = scratch_for_device(&work))) return rc;
  const int chunk = (int)std::min<size_t>((size_t)H, SFFFT_SCRATCH_BYTES / per);
  for (int h0 = 0; h0 < H; h0 += chunk)
    if ((rc = spectrum_impl(k, nullptr, std::min(chunk, H - h0), L, L, plan, kf, work, stream, 0, 0, h0)))
      return rc;
  return SFFFT_OK;
}

int sffft_spectrum_complex(const float* kr, const float* ki, int H, int L, const sffft_plan* plan, void* kf,
                           void* work, void* stream) {
  // pairs of sequences per transform only: they carry the real and imaginary planes of u and y
  if (!plan || plan->seqs != 2 || !ki || ki == kr) return SFFFT_EINVAL;
  return spectrum_impl(kr, ki, H, L, L, plan, kf, work, stream, 1);
}

int sffft_spectrum_circular(const float* k, int H, int N, const sffft_plan* plan, void* kf, void* work,
                            void* stream) {
  if (N < 2 || N % 2 || !plan || plan->mode != 2) return SFFFT_EINVAL;
  return spectrum_impl(k, nullptr, H, N / 2, N, plan, kf, work, stream);
}

int sffft_circconv_long_f32(const float* u, const void* kf, float* y, void* work, size_t work_bytes, int B, int H,
                            int N, const sffft_plan* plan, void* stream) {
  if (N < 2 || N % 2) return SFFFT_EINVAL;
  return conv_long<0>(u, kf, y, work, work_bytes, B, H, N / 2, plan, stream, 1);
}

int sffft_circconv_long_bf16(const uint16_t* u, const void* kf, uint16_t* y, void* work, size_t work_bytes, int B,
                             int H, int N, const sffft_plan* plan, void* stream) {
  if (N < 2 || N % 2) return SFFFT_EINVAL;
  return conv_long<1>(u, kf, y, work, work_bytes, B, H, N / 2, plan, stream, 1);
}

int sffft_spectrum_from_natural(const void* kc, int H, int L, const sffft_plan* plan, void* kf, void* stream) {
  if (!kc || !kf || H < 1 || kc == kf) return SFFFT_EINVAL;
  const int rc = check_shape(L, plan);
  if (rc) return rc;
  return permute_launch(static_cast<const float2*>(kc), static_cast<float2*>(kf), H, plan, 0, 0,
                        (hipStream_t)stream);
}

int sffft_spectrum_from_natural_complex(const void* kc, int H, int L, const sffft_plan* plan, void* kf,
                                        void* stream) {
  if (!kc || !kf || H < 1 || kc == kf || !plan || plan->seqs != 2) return SFFFT_EINVAL;
  const int rc = check_shape(L, plan);
  if (rc) return rc;
  return permute_launch(static_cast<const float2*>(kc), static_cast<float2*>(kf), H, plan, 1, 0,
                        (hipStream_t)stream);
}

int sffft_conv_f32(const float* u, const void* kf, float* y, int B, int H, int L, const sffft_plan* plan,
                   void* stream) {
  return conv<0>(u, kf, y, B, H, L, plan, stream);
}

int sffft_conv_bf16(const uint16_t* u, const void* kf, uint16_t* y, int B, int H, int L, const sffft_plan* plan,
                    void* stream) {
  return conv<1>(u, kf, y, B, H, L, plan, stream);
}

int sffft_conv_complex_f32(const float* u, const void* kf, float* y, int B, int H, int L, const sffft_plan* plan,
                           void* stream) {
  if (!plan || plan->seqs != 2 || plan->acc != 0 || plan->mode == 2) return SFFFT_EINVAL;
  return conv<0>(u, kf, y, B, H, L, plan, stream, 1);
}

int sffft_conv_complex_bf16(const uint16_t* u, const void* kf, uint16_t* y, int B, int H, int L,
                            const sffft_plan* plan, void* stream) {
  if (!plan || plan->seqs != 2 || plan->acc != 0 || plan->mode == 2) return SFFFT_EINVAL;
  return conv<1>(u, kf, y, B, H, L, plan, stream, 1);
}

size_t sffft_work_bytes(int B, int H, int L, const sffft_plan* plan) {
  if (B < 2 || B % 2 || H < 1 || check_shape(L, plan) || plan->mode != 2) return 0;
  return work_bytes(B, H, L);
}

int sffft_conv_long_f32(const float* u, const void* kf, float* y, void* work, size_t work_bytes, int B, int H, int L,
                        const sffft_plan* plan, void* stream) {
  return conv_long<0>(u, kf, y, work, work_bytes, B, H, L, plan, stream);
}

int sffft_conv_long_bf16(const uint16_t* u, const void* kf, uint16_t* y, void* work, size_t work_bytes, int B, int H,
                         int L, const sffft_plan* plan, void* stream) {
  return conv_long<1>(u, kf, y, work, work_bytes, B, H, L, plan, stream);
}

int sffft_dispatch_floor(int B, int H, int L, const sffft_plan* plan, void* stream) {
  if (B < 1 || H < 1 || (long long)B * H > INT_MAX) return SFFFT_EINVAL;
  int rc = check_shape(L, plan);
  if (rc) return rc;
  if (B % plan->seqs || plan->mode == 2) return SFFFT_EINVAL;
  const Entry* e = find_entry(L, plan);
  if (!e) return SFFFT_ENOPLAN;
  const unsigned grid = e->mode == 1 ? (unsigned)((H + e->channels - 1) / e->channels)
                                     : (unsigned)(H * (B / plan->seqs));
  return sffft_dispatch_floor_shape(grid, 64u * (unsigned)plan->waves, (unsigned)e->lds_bytes, stream);
}

int sffft_dispatch_floor_shape(unsigned grid, unsigned block, unsigned lds_bytes, void* stream) {
  if (grid < 1 || block < 64 || block > 1024 || block % 64 || lds_bytes > 163840) return SFFFT_EINVAL;
  static std::once_flag attr_once;
  static int attr_rc = SFFFT_OK;
  std::call_once(attr_once, [] {
    attr_rc = hip_status(hipFuncSetAttribute(reinterpret_cast<const void*>(&empty_dispatch_kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, 163840),
                         "hipFuncSetAttribute");
  });
  if (attr_rc) return attr_rc;
  hipLaunchKernelGGL(empty_dispatch_kernel, dim3(grid), dim3(block), lds_bytes, (hipStream_t)stream);
  return hip_status(hipGetLastError(), "dispatch floor launch");
}

namespace {
bool span_overlap(const void* a, size_t na, const void* b, size_t nb) {
  const uintptr_t x = (uintptr_t)a, z = (uintptr_t)b;
  return na && nb && x < z + nb && z < x + na;
}
bool aligned8(const void* p) { return ((uintptr_t)p & 7u) == 0; }

// Validated 1-D transform layout; *extent: extent of x / X in complex elements. Two layout
// families are supported, both one-to-one (no two (sequence, element) pairs at one
// address): each sequence whole before the next (dist >= N * stride), or the sequences
// interleaved within one element step (stride >= batch * dist), as the columns of a
// row-major matrix are. Other layouts are rejected, also the non-overlapping ones between
// the two families (batch 3, N 4, stride 2, dist 5 is one).
int fft_layout(int batch, int N, long long stride, long long dist, xf::Seqs* q, long long* extent) {
  xf::Radices d;
  if (batch < 1 || !xf::split(N, &d) || (long long)batch * N > xf::MAX_ELEMS) return SFFFT_EINVAL;
  if (stride < 1 || dist < 0 || (batch > 1 && dist < 1)) return SFFFT_EINVAL;
  if (batch > 1 && stride > ((long long)1 << 40) / N) return SFFFT_EINVAL;  // keeps N * stride in range
  if (batch > 1 && dist < (long long)N * stride && stride < (long long)batch * dist) return SFFFT_EINVAL;
  *q = xf::Seqs{batch, batch, dist, 0, stride, dist < stride ? 1 : 0};
  *extent = (long long)(batch - 1) * dist + (long long)(N - 1) * stride + 1;
  return SFFFT_OK;
}

int fft2_layout(int batch, int N0, int N1, long long* elems, long long* work) {
  xf::Radices d;
  if (batch < 1 || !xf::split(N0, &d) || !xf::split(N1, &d)) return SFFFT_EINVAL;
  const long long n = (long long)batch * N0 * N1;
  if (n > xf::MAX_ELEMS) return SFFFT_EINVAL;
  *elems = n;
  *work = xf::work2_elems(batch, N0, N1);
  return SFFFT_OK;
}

int circconv2d_layout(int B, int H, int N0, int N1, long long* elems, long long* work) {
  xf::Radices d;
  if (B < 1 || H < 1 || !xf::split(N0, &d) || !xf::split(N1, &d)) return SFFFT_EINVAL;
  const long long n = (long long)B * H * N0 * N1;
  if (n > xf::MAX_ELEMS) return SFFFT_EINVAL;
  *elems = n;
  *work = xf::circconv2d_elems(B, H, N0, N1);
  return SFFFT_OK;
}
}  // namespace

size_t sffft_fft_work_bytes(int batch, int N) {
  xf::Seqs q;
  long long ext;
  if (fft_layout(batch, N, 1, N, &q, &ext)) return 0;
  return (size_t)xf::work_elems(q, N) * 8;
}

int sffft_fft_c2c(const void* x, void* X, void* work, size_t work_bytes, int batch, int N, long long stride,
                  long long dist, int inverse, float scale, void* stream) {
  xf::Seqs q;
  long long ext;
  if (!x || !X || !aligned8(x) || !aligned8(X) || (inverse != 0 && inverse != 1)) return SFFFT_EINVAL;
  if (fft_layout(batch, N, stride, dist, &q, &ext)) return SFFFT_EINVAL;
  // in place (x == X) or disjoint; a partial overlap would let one stage overwrite input
  // another thread has yet to read
  if (x != X && span_overlap(x, (size_t)ext * 8, X, (size_t)ext * 8)) return SFFFT_EINVAL;
  const size_t need = (size_t)xf::work_elems(q, N) * 8;
  if (need && (!work || !aligned8(work) || work_bytes < need || span_overlap(work, need, x, ext * 8) ||
               span_overlap(work, need, X, ext * 8)))
    return SFFFT_EINVAL;
  return hip_status(xf::run(static_cast<const float2*>(x), static_cast<float2*>(X), static_cast<float2*>(work), q, N,
                            inverse, scale, (hipStream_t)stream),
                    "fft launch");
}

size_t sffft_fft2_work_bytes(int batch, int N0, int N1) {
  long long n, w;
  if (fft2_layout(batch, N0, N1, &n, &w)) return 0;
  return (size_t)w * 8;
}

int sffft_fft2_c2c(const void* x, void* X, void* work, size_t work_bytes, int batch, int N0, int N1, int inverse,
                   float scale, void* stream) {
  long long n, w;
  if (!x || !X || !aligned8(x) || !aligned8(X) || (inverse != 0 && inverse != 1)) return SFFFT_EINVAL;
  if (fft2_layout(batch, N0, N1, &n, &w)) return SFFFT_EINVAL;
  const size_t need = (size_t)w * 8, bytes = (size_t)n * 8;
  if (x != X && span_overlap(x, bytes, X, bytes)) return SFFFT_EINVAL;  // partial overlap
  if (need && (!work || !aligned8(work) || work_bytes < need || span_overlap(work, need, x, bytes) ||
               span_overlap(work, need, X, bytes)))
    return SFFFT_EINVAL;
  return hip_status(xf::run2(static_cast<const float2*>(x), static_cast<float2*>(X), static_cast<float2*>(work), batch,
                             N0, N1, inverse, scale, (hipStream_t)stream),
                    "fft2 launch");
}

size_t sffft_circconv2d_work_bytes(int B, int H, int N0, int N1) {
  long long n, w;
  if (circconv2d_layout(B, H, N0, N1, &n, &w)) return 0;
  return (size_t)w * 8;
}

int sffft_circconv2d_f32(const float* u, const float* k, float* y, void* work, size_t work_bytes, int B, int H,
                         int N0, int N1, void* stream) {
  long long n, w;
  if (!u || !k || !y || !work || !aligned16(u) || !aligned16(k) || !aligned16(y) || !aligned16(work))
    return SFFFT_EINVAL;
  if (circconv2d_layout(B, H, N0, N1, &n, &w)) return SFFFT_EINVAL;
  const size_t need = (size_t)w * 8, io = (size_t)n * 4, kb = (size_t)H * N0 * N1 * 4;
  if (work_bytes < need || span_overlap(work, need, u, io) || span_overlap(work, need, y, io) ||
      span_overlap(work, need, k, kb) || span_overlap(y, io, u, io) || span_overlap(y, io, k, kb))
    return SFFFT_EINVAL;
  return hip_status(xf::circconv2d(u, k, y, static_cast<float2*>(work), B, H, N0, N1, (hipStream_t)stream),
                    "circconv2d launch");
}

int sffft_to_bf16(const float* x, uint16_t* y, size_t n, void* stream) {
  if (!x || !y) return SFFFT_EINVAL;
  if (!n) return SFFFT_OK;
  hipLaunchKernelGGL(to_bf16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, x, y, n);
  return hip_status(hipGetLastError(), "to_bf16 launch");
}

int sffft_dft_table(void* out, size_t out_len) {
  const size_t bytes = (size_t)FTAB_H8 * 16;
  if (!out || out_len < bytes) return SFFFT_EINVAL;
  const void* table = nullptr;
  const int rc = device_table(&table);
  if (rc) return rc;
  return hip_status(hipMemcpy(out, table, bytes, hipMemcpyDeviceToHost), "hipMemcpy");
}

int sffft_twiddle_probe(int N, const void* queries, int nq, int rows, float sc, void* out, void* stream) {
  if (!queries || !out || nq < 1 || rows < 0 || rows > 64) return SFFFT_EINVAL;
  const dim3 grid((unsigned)((nq + 63) / 64)), block(64);
  const int4* q = static_cast<const int4*>(queries);
  float2* o = static_cast<float2*>(out);
  hipStream_t s = (hipStream_t)stream;
  switch (N) {
    case 256: hipLaunchKernelGGL(twiddle_probe_kernel<256>, grid, block, 0, s, q, o, nq, rows, sc); break;
    case 512: hipLaunchKernelGGL(twiddle_probe_kernel<512>, grid, block, 0, s, q, o, nq, rows, sc); break;
    case 1024: hipLaunchKernelGGL(twiddle_probe_kernel<1024>, grid, block, 0, s, q, o, nq, rows, sc); break;
    case 2048: hipLaunchKernelGGL(twiddle_probe_kernel<2048>, grid, block, 0, s, q, o, nq, rows, sc); break;
    case 4096: hipLaunchKernelGGL(twiddle_probe_kernel<4096>, grid, block, 0, s, q, o, nq, rows, sc); break;
    case 8192: hipLaunchKernelGGL(twiddle_probe_kernel<8192>, grid, block, 0, s, q, o, nq, rows, sc); break;
    case 16384: hipLaunchKernelGGL(twiddle_probe_kernel<16384>, grid, block, 0, s, q, o, nq, rows, sc); break;
    case 32768: hipLaunchKernelGGL(twiddle_probe_kernel<32768>, grid, block, 0, s, q, o, nq, rows, sc); break;
    default: return SFFFT_EINVAL;
  }
  return hip_status(hipGetLastError(), "twiddle probe launch");
}

int sffft_twiddle_table(int r0, int r1, int layout, void* out, size_t out_len) {
  if (!valid_radix(r0) || !valid_radix(r1) || layout < 0 || layout > 2 || !out) return SFFFT_EINVAL;
  const size_t bytes = (size_t)r0 * r1 * (layout == 2 ? 8 : 16);  // two tables of N complex fp32 / fp16
  if (out_len < bytes) return SFFFT_EINVAL;
  const void* tw = nullptr;
  const int rc = device_twiddles(r0, r1, layout, &tw);
  if (rc) return rc;
  return hip_status(hipMemcpy(out, tw, bytes, hipMemcpyDeviceToHost), "hipMemcpy");
}

int sffft_select_candidate(const sffft_candidate* c, int n, double max_error, const char* io) {
  if (!std::isfinite(max_error) || max_error <= 0 || !io) return -1;
  if (std::strcmp(io, "fp32") && std::strcmp(io, "bf16") && std::strcmp(io, "any")) return -1;
  int best = -1;
  for (int i = 0; i < n; i++) {
    if (!c || !c[i].io) continue;
    if (std::strcmp(io, "any") && std::strcmp(io, c[i].io)) continue;
    const double ms = c[i].ms, err = c[i].rel_err;
    if (!std::isfinite(ms) || ms <= 0 || !std::isfinite(err) || err < 0 || err > max_error) continue;
    if (best < 0 || ms < c[best].ms || (ms == c[best].ms && err < c[best].rel_err)) best = i;
  }
  return best;
}

double sffft_relative_l2(double squared_error, double squared_reference) {
  if (squared_reference > 0) return std::sqrt(squared_error / squared_reference);
  return squared_error == 0 ? 0.0 : std::numeric_limits<double>::infinity();
}

const char* sffft_last_error(void) { return g_last_error; }

const char* sffft_strerror(int code) {
  switch (code) {
    case SFFFT_OK: return "success";
    case SFFFT_EINVAL: return "invalid argument";
    case SFFFT_ENOPLAN: return "plan not compiled into this library";
    case SFFFT_EHIP: return "HIP runtime error";
    case SFFFT_ENOTFOUND: return "not found";
    case SFFFT_ESCRATCH: return "the call needs more workspace than the library's static scratch holds";
    default: return "unknown error";
  }
}

}  // extern "C"
