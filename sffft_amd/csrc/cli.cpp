// `sffft` driver: the reference's benchmark/selector CLI on MI355X.
//
//   sffft [B H [L]] [--max-error REL_L2] [--io fp32|bf16|any] [--seed N]
//         [--input-scale S] [--allocator device|managed|mapped|hybrid]
//         [--kernel legacy|cached|auto] [--memory-info]
//
// Same grammar, validation, exit codes (0 ok, 1 invalid arguments, 2 no match)
// and CSV lines as the reference driver (src/sffft.cu:423-515). Per length it
// times the rocFFT pipeline (the comparator; the reference used cuFFT), every
// compiled fused plan with fp32 and fp16 accumulation and fp32 and bf16 I/O, and
// prints RESULT,L,method,config,ms,rel_err lines; --max-error selects the fastest
// candidate within the error budget (src/selection.h semantics via the C ABI).
// Differences: L may also be 16384 (L=0 still sweeps 128..8192); "w" in the config
// counts 64-lane wavefronts; the config ends with /seq<n> (rows per transform) and
// /wg or /wave<c> (one workgroup per transform, or one wavefront per transform
// with c channels per workgroup).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cerrno>
#include <chrono>
#include <climits>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <set>
#include <string>
#include <tuple>
#include <vector>

#include "../../include/sffft.h"
#include "rocfft_pipeline.h"

#define HK(x)                                                                                 \
  do {                                                                                        \
    hipError_t e_ = (x);                                                                      \
    if (e_ != hipSuccess) {                                                                   \
      printf("HIP %s @%d: %s\n", #x, __LINE__, hipGetErrorString(e_));                        \
      exit(1);                                                                                \
    }                                                                                         \
  } while (0)
#define SK(x)                                                                                 \
  do {                                                                                        \
    int r_ = (x);                                                                             \
    if (r_ != SFFFT_OK) {                                                                     \
      printf("sffft %s @%d: %s %s\n", #x, __LINE__, sffft_strerror(r_), sffft_last_error()); \
      exit(1);                                                                                \
    }                                                                                         \
  } while (0)

namespace {

using Clock = std::chrono::steady_clock;
double elapsed_ms(Clock::time_point t0) {
  return std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
}

// ---- buffers: device, managed, mapped host, or hybrid (src/sffft.cu:25-86) ------
enum class Alloc { Device, Managed, Mapped, Hybrid };
const char* alloc_name(Alloc a) {
  return a == Alloc::Device ? "device" : a == Alloc::Managed ? "managed" : a == Alloc::Mapped ? "mapped" : "hybrid";
}

struct Buffers {
  struct Block {
    void* dev;
    void* host;
    size_t bytes;
    Alloc kind;
  };
  Alloc mode;
  bool can_prefetch;
  std::vector<Block> blocks;
  size_t owned = 0, uploaded = 0, downloaded = 0;
  double alloc_ms = 0, copy_ms = 0;
  Buffers(Alloc m, bool prefetch) : mode(m), can_prefetch(prefetch) {}
  Buffers(const Buffers&) = delete;
  Buffers& operator=(const Buffers&) = delete;
  // shared_io: the buffer is an input/output the host touches (mapped in hybrid mode)
  template <class T>
  T* get(size_t count, bool shared_io = true) {
    const size_t bytes = count * sizeof(T);
    const Alloc kind = mode == Alloc::Hybrid ? (shared_io ? Alloc::Mapped : Alloc::Device) : mode;
    auto t0 = Clock::now();
    void* d = nullptr;
    void* h = nullptr;
    if (kind == Alloc::Mapped) {
      HK(hipHostMalloc(&h, bytes, hipHostMallocMapped));
      HK(hipHostGetDevicePointer(&d, h, 0));
    } else if (kind == Alloc::Managed) {
      HK(hipMallocManaged(&d, bytes));
      h = d;
    } else {
      HK(hipMalloc(&d, bytes));
    }
    blocks.push_back({d, h, bytes, kind});
    owned += bytes;
    alloc_ms += elapsed_ms(t0);
    return static_cast<T*>(d);
  }
  template <class T>
  T* host_view(const T* dev) {
    for (auto& b : blocks)
      if (b.dev == dev) return static_cast<T*>(b.host);
    return nullptr;
  }
  void prefetch(const void* p, size_t bytes, bool to_gpu) {
    if (mode != Alloc::Managed || !can_prefetch) return;
    int dev = 0;
    HK(hipGetDevice(&dev));
    HK(hipMemPrefetchAsync(p, bytes, to_gpu ? dev : hipCpuDeviceId, nullptr));
  }
  void to_gpu() {
    for (auto& b : blocks) prefetch(b.dev, b.bytes, true);
  }
  template <class T>
  void upload(T* dev, const T* src, size_t count) {
    T* h = host_view(dev);
    if (h == src) return;
    auto t0 = Clock::now();
    if (h) {
      std::memcpy(h, src, count * sizeof(T));
    } else {
      HK(hipMemcpy(dev, src, count * sizeof(T), hipMemcpyHostToDevice));
      uploaded += count * sizeof(T);
    }
    copy_ms += elapsed_ms(t0);
  }
  // Host-readable contents of a device buffer: its host view when it has one,
  // else a copy into `shadow`.
  template <class T>
  const T* read(const T* dev, size_t count, std::vector<T>& shadow) {
    if (T* h = host_view(dev)) {
      prefetch(dev, count * sizeof(T), false);
      HK(hipDeviceSynchronize());
      return h;
    }
    shadow.resize(count);
    auto t0 = Clock::now();
    HK(hipMemcpy(shadow.data(), dev, count * sizeof(T), hipMemcpyDeviceToHost));
    downloaded += count * sizeof(T);
    copy_ms += elapsed_ms(t0);
    return shadow.data();
  }
  ~Buffers() {
    for (auto& b : blocks) {
      if (b.kind == Alloc::Mapped)
        (void)hipHostFree(b.host);
      else
        (void)hipFree(b.dev);
    }
  }
};

// ---- input generator (src/sffft.cu:308-310, 339-341) ----------------------------
uint64_t g_rng = 88172645463325252ULL;
double urand() {
  g_rng ^= g_rng << 13;
  g_rng ^= g_rng >> 7;
  g_rng ^= g_rng << 17;
  return ((g_rng >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}
// The reference's `sqrt(-2*log(urand()))*cos(2*M_PI*urand())` leaves the order of
// the two calls unspecified; GCC and clang take the log argument first.
double nrand() {
  const double u1 = urand();
  const double u2 = urand();
  return std::sqrt(-2 * std::log(u1)) * std::cos(2 * M_PI * u2);
}

// The calibration inputs of one length, drawn from the running generator state:
// u [BH][L] ~ N(0,1) * input_scale in (b, h, n) order, then k [H][L] with the decay
// a = 1 / (4 + L h / H) (src/sffft.cu:339-341).
void generate_inputs(size_t BH, int H, int L, double input_scale, float* u, float* k) {
  for (size_t i = 0; i < BH * L; i++) u[i] = (float)(nrand() * input_scale);
  for (int h = 0; h < H; h++) {
    const double a = 1.0 / (4.0 + (double)L * h / H);
    for (int n = 0; n < L; n++) k[(size_t)h * L + n] = (float)(nrand() * std::exp(-a * n) * std::sqrt(2 * a));
  }
}

uint16_t bf16_bits(float f) {  // round to nearest even (the device conversion's rule)
  uint32_t x;
  std::memcpy(&x, &f, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}
float bf16_value(uint16_t b) {
  const uint32_t x = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &x, 4);
  return f;
}

struct Candidate {
  std::string method, io, config;
  double ms, rel_err;
};

struct Bench {
  int L, N, H, B;
  size_t BH;
  int iters;
  Buffers mem;
  std::vector<float> hu_shadow, hk, yref_shadow;
  float* hu = nullptr;
  const float* yref = nullptr;
  double setup_ms = 0;
  std::vector<Candidate> candidates;
  float *du, *dy, *dyref, *dk;
  uint16_t *dub, *dyb;
  void *dkc, *dkf;
  sffft_rocfft* fft = nullptr;
  hipEvent_t e0, e1;
  int kernel_mode;

  template <class F>
  float timeit(F f) {  // src/sffft.cu:321-324
    for (int i = 0; i < 3; i++) f();
    HK(hipDeviceSynchronize());
    HK(hipEventRecord(e0, nullptr));
    for (int i = 0; i < iters; i++) f();
    HK(hipEventRecord(e1, nullptr));
    HK(hipEventSynchronize(e1));
    float ms = 0;
    HK(hipEventElapsedTime(&ms, e0, e1));
    HK(hipGetLastError());
    return ms / iters;
  }

  Bench(int L_, int B_, int H_, double input_scale, Alloc mode, bool can_prefetch, int kernel_mode_)
      : L(L_), N(2 * L_), H(H_), B(B_), BH((size_t)B_ * H_), mem(mode, can_prefetch), kernel_mode(kernel_mode_) {
    auto t0 = Clock::now();
    iters = std::min(200, std::max(10, 20000 / L));
    du = mem.get<float>(BH * L);
    dy = mem.get<float>(BH * L);
    dyref = mem.get<float>(BH * L);
    dub = mem.get<uint16_t>(BH * L, false);
    dyb = mem.get<uint16_t>(BH * L);
    dk = mem.get<float>((size_t)H * L);
    dkc = mem.get<float>((size_t)H * N * 2, false);
    dkf = mem.get<float>((size_t)H * N * 2, false);
    hu = mem.host_view(du);
    if (!hu) {
      hu_shadow.resize(BH * L);
      hu = hu_shadow.data();
    }
    float* hkv = mem.host_view(dk);
    hk.resize((size_t)H * L);
    generate_inputs(BH, H, L, input_scale, hu, hk.data());
    if (hkv) std::memcpy(hkv, hk.data(), hk.size() * 4);
    mem.upload(du, hu, BH * L);
    if (!hkv) mem.upload(dk, hk.data(), hk.size());
    mem.to_gpu();
    SK(sffft_to_bf16(du, dub, BH * L, nullptr));
    if (sffft_rocfft_create(B, H, L, nullptr, &fft)) {
      printf("rocFFT plan creation failed\n");
      exit(1);
    }
    if (sffft_rocfft_filter(fft, dk, dkc)) {
      printf("rocFFT filter spectrum failed\n");
      exit(1);
    }
    HK(hipEventCreate(&e0));
    HK(hipEventCreate(&e1));
    HK(hipDeviceSynchronize());
    setup_ms = elapsed_ms(t0);
  }
  ~Bench() {
    sffft_rocfft_destroy(fft);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
  }

  // rocFFT pipeline (the reference's cuFFT baseline, src/sffft.cu:370-381): timed,
  // then checked against an fp64 direct convolution of 3 sequences.
  void baseline() {
    auto full = [&] {
      if (sffft_rocfft_full(fft, du, dyref)) {
        printf("rocFFT pipeline failed\n");
        exit(1);
      }
    };
    auto core = [&] {
      if (sffft_rocfft_core(fft)) {
        printf("rocFFT core failed\n");
        exit(1);
      }
    };
    const float t_full = timeit(full), t_core = timeit(core);
    full();
    HK(hipDeviceSynchronize());
    yref = mem.read(dyref, BH * L, yref_shadow);
    double rn = 0, rd = 0;
    for (size_t s : {(size_t)0, BH / 2, BH - 1}) {
      const int h = (int)(s % H);
      for (int n = 0; n < L; n++) {
        double acc = 0;
        for (int m = 0; m <= n; m++) acc += (double)hu[s * L + m] * hk[(size_t)h * L + n - m];
        const double d = yref[s * L + n] - acc;
        rn += d * d;
        rd += acc * acc;
      }
    }
    const double err = sffft_relative_l2(rn, rd);
    printf("RESULT,%d,rocfft_pipeline_fp32,-,%.5f,%.3e\n", L, t_full, err);
    printf("RESULT,%d,rocfft_core_fp32,-,%.5f,%.3e\n", L, t_core, err);
    fflush(stdout);
  }

  // One compiled plan with one accumulation type and DFT-matrix source
  // (src/sffft.cu:382-405).
  void fused(const sffft_plan& p, const char* name) {
    int occ = 0;
    SK(sffft_plan_occupancy(L, &p, &occ));
    const size_t lds = sffft_plan_lds_bytes(L, &p);
    auto f32 = [&] { SK(sffft_conv_f32(du, dkf, dy, B, H, L, &p, nullptr)); };
    auto b16 = [&] { SK(sffft_conv_bf16(dub, dkf, dyb, B, H, L, &p, nullptr)); };
    const float t32 = timeit(f32), t16 = timeit(b16);
    f32();
    HK(hipDeviceSynchronize());
    std::vector<float> y_shadow;
    const float* y = mem.read(dy, BH * L, y_shadow);
    std::vector<uint16_t> yb_shadow;
    b16();
    HK(hipDeviceSynchronize());
    const uint16_t* yb = mem.read(dyb, BH * L, yb_shadow);
    double n1 = 0, n2 = 0, d = 0;
    for (size_t i = 0; i < BH * L; i++) {
      const double r = yref[i], a = y[i] - r, b = (double)bf16_value(yb[i]) - r;
      n1 += a * a;
      n2 += b * b;
      d += r * r;
    }
    char config[128];
    char mode[16];
    if (p.mode)
      snprintf(mode, sizeof(mode), "wave%d", p.channels);
    else
      snprintf(mode, sizeof(mode), "wg");
    snprintf(config, sizeof(config), "%s/w%d/occ%d/smem%zu/kernel_%s/seq%d/%s", name, p.waves, occ, lds,
             p.cached ? "cached" : "legacy", p.seqs, mode);
    const char* m32 = p.acc ? "fused_fp16acc_fp32io" : "fused_fp32io";
    const char* m16 = p.acc ? "fused_fp16acc_bf16io" : "fused_bf16io";
    const double err32 = sffft_relative_l2(n1, d), err16 = sffft_relative_l2(n2, d);
    candidates.push_back({m32, "fp32", config, t32, err32});
    candidates.push_back({m16, "bf16", config, t16, err16});
    printf("RESULT,%d,%s,%s,%.5f,%.3e\n", L, m32, config, t32, err32);
    printf("RESULT,%d,%s,%s,%.5f,%.3e\n", L, m16, config, t16, err16);
    fflush(stdout);
  }

  // Every compiled plan for L, both accumulation types, legacy and/or cached DFT
  // matrices (src/sffft.cu:406-409, 507-513).
  void variants() {
    std::tuple<int, int, int, int> spectrum_of = {0, 0, 0, -1};
    const int n = sffft_plan_count(L);
    for (int i = 0; i < n; i++) {
      sffft_plan p;
      char name[32];
      SK(sffft_plan_get(L, i, &p, name, sizeof(name)));
      if (B % p.seqs) continue;
      const std::tuple<int, int, int, int> radices = {p.r0, p.r1, p.r2, p.mode};  // spectrum order
      if (radices != spectrum_of) {  // kernel-order spectrum from the rocFFT C2C spectrum (permuteK)
        SK(sffft_spectrum_from_natural(dkc, H, L, &p, dkf, nullptr));
        spectrum_of = radices;
      }
      for (int cached = 0; cached < 2; cached++) {
        if ((kernel_mode == 0 && cached) || (kernel_mode == 1 && !cached)) continue;
        for (int acc = 0; acc < 2; acc++) {
          p.cached = cached;
          p.acc = acc;
          fused(p, name);
        }
      }
    }
  }

  bool select(double max_error, const char* io) {  // src/sffft.cu:410-415
    std::vector<sffft_candidate> c;
    for (auto& x : candidates) c.push_back({x.method.c_str(), x.io.c_str(), x.config.c_str(), x.ms, x.rel_err});
    const int best = sffft_select_candidate(c.data(), (int)c.size(), max_error, io);
    if (best < 0) {
      printf("NO_MATCH,%d,%s,%.9e\n", L, io, max_error);
      return false;
    }
    const Candidate& b = candidates[best];
    printf("SELECT,%d,%s,%s,%.5f,%.9e,%.9e,%s\n", L, b.method.c_str(), b.config.c_str(), b.ms, b.rel_err,
           max_error, b.io.c_str());
    return true;
  }

  void report_memory() {  // src/sffft.cu:416-419
    printf("MEMORY,%d,%s,%zu,%zu,%.3f,%zu,%zu,%.3f,%.3f\n", L, alloc_name(mem.mode), mem.owned,
           (hu_shadow.size() + yref_shadow.size()) * sizeof(float), mem.alloc_ms, mem.uploaded, mem.downloaded,
           mem.copy_ms, setup_ms);
  }
};

void usage() {
  printf(
      "Usage: sffft [B H [L]] [--max-error REL_L2] [--io fp32|bf16|any] [--seed N] [--input-scale SCALE] "
      "[--allocator device|managed|mapped|hybrid] [--kernel legacy|cached|auto] [--memory-info] "
      "[--dump-inputs FILE]\n"
      "L: 0 (all of 128..8192) or a power of two from 128 to 16384. Defaults: B=8 H=768, io=fp32.\n"
      "--max-error selects the fastest passing fused plan on these calibration inputs.\n"
      "Error is measured against the rocFFT fp32 pipeline; no match exits 2. Invalid arguments exit 1.\n"
      "--dump-inputs writes the calibration inputs of length L (u [B][H][L] then k [H][L], raw fp32)\n"
      "to FILE and exits without touching the GPU (needs L).\n");
}

}  // namespace

int main(int argc, char** argv) {
  int B = 8, H = 768, only = 0, positional = 0, failed = 0;
  double max_error = -1, input_scale = 1;
  const char* io = "fp32";
  Alloc allocation = Alloc::Device;
  bool memory_info = false;
  const char* dump_path = nullptr;
  int kernel_mode = 0;  // 0 legacy, 1 cached, 2 auto
  for (int i = 1; i < argc; i++) {
    const char* arg = argv[i];
    char* end = nullptr;
    errno = 0;
    if (!strcmp(arg, "--help") || !strcmp(arg, "-h")) {
      usage();
      return 0;
    }
    if (!strcmp(arg, "--memory-info")) {
      memory_info = true;
      continue;
    }
    if (!strcmp(arg, "--dump-inputs")) {
      if (++i == argc) {
        usage();
        return 1;
      }
      dump_path = argv[i];
      continue;
    }
    if (!strcmp(arg, "--allocator")) {
      if (++i == argc) {
        usage();
        return 1;
      }
      if (!strcmp(argv[i], "device"))
        allocation = Alloc::Device;
      else if (!strcmp(argv[i], "managed"))
        allocation = Alloc::Managed;
      else if (!strcmp(argv[i], "mapped"))
        allocation = Alloc::Mapped;
      else if (!strcmp(argv[i], "hybrid"))
        allocation = Alloc::Hybrid;
      else {
        fprintf(stderr, "--allocator must be device, managed, mapped, or hybrid\n");
        return 1;
      }
    } else if (!strcmp(arg, "--kernel")) {
      if (++i == argc) {
        usage();
        return 1;
      }
      if (!strcmp(argv[i], "legacy"))
        kernel_mode = 0;
      else if (!strcmp(argv[i], "cached"))
        kernel_mode = 1;
      else if (!strcmp(argv[i], "auto"))
        kernel_mode = 2;
      else {
        fprintf(stderr, "--kernel must be legacy, cached, or auto\n");
        return 1;
      }
    } else if (!strcmp(arg, "--max-error")) {
      if (++i == argc) {
        usage();
        return 1;
      }
      max_error = strtod(argv[i], &end);
      if (errno || end == argv[i] || *end || !std::isfinite(max_error) || max_error <= 0) {
        fprintf(stderr, "--max-error must be positive and finite\n");
        return 1;
      }
    } else if (!strcmp(arg, "--input-scale")) {
      if (++i == argc) {
        usage();
        return 1;
      }
      input_scale = strtod(argv[i], &end);
      if (errno || end == argv[i] || *end || !std::isfinite(input_scale) || input_scale <= 0 ||
          input_scale > std::numeric_limits<float>::max()) {
        fprintf(stderr, "--input-scale must be positive, finite, and representable in fp32\n");
        return 1;
      }
    } else if (!strcmp(arg, "--io")) {
      if (++i == argc) {
        usage();
        return 1;
      }
      io = argv[i];
      if (strcmp(io, "fp32") && strcmp(io, "bf16") && strcmp(io, "any")) {
        fprintf(stderr, "--io must be fp32, bf16, or any\n");
        return 1;
      }
    } else if (!strcmp(arg, "--seed")) {
      if (++i == argc) {
        usage();
        return 1;
      }
      g_rng = strtoull(argv[i], &end, 10);
      if (errno || end == argv[i] || *end || argv[i][0] == '-' || !g_rng) {
        fprintf(stderr, "--seed must be a nonzero unsigned integer\n");
        return 1;
      }
    } else {
      const long value = strtol(arg, &end, 10);
      if (errno || end == arg || *end || value < 0 || value > INT_MAX || positional == 3) {
        fprintf(stderr, "Invalid argument: %s\n", arg);
        usage();
        return 1;
      }
      if (positional == 0)
        B = (int)value;
      else if (positional == 1)
        H = (int)value;
      else
        only = (int)value;
      positional++;
    }
  }
  if (B < 1 || H < 1 || (long long)B * H > INT_MAX ||
      (only && (only < 128 || only > 16384 || (only & (only - 1))))) {
    fprintf(stderr,
            "B and H must be positive with B*H <= INT_MAX; L must be 0 or 128,256,512,1024,2048,4096,8192,16384\n");
    return 1;
  }
  if (dump_path) {  // host only: the inputs the run of length `only` would use
    if (!only) {
      fprintf(stderr, "--dump-inputs needs L\n");
      return 1;
    }
    const size_t BH = (size_t)B * H;
    std::vector<float> hu(BH * only), hk((size_t)H * only);
    generate_inputs(BH, H, only, input_scale, hu.data(), hk.data());
    FILE* f = fopen(dump_path, "wb");
    if (!f || fwrite(hu.data(), 4, hu.size(), f) != hu.size() || fwrite(hk.data(), 4, hk.size(), f) != hk.size() ||
        fclose(f)) {
      fprintf(stderr, "--dump-inputs: cannot write %s\n", dump_path);
      return 1;
    }
    return 0;
  }
  hipDeviceProp_t p;
  HK(hipGetDeviceProperties(&p, 0));
  int managed = 0, concurrent = 0, pageable = 0, host_tables = 0;
  HK(hipDeviceGetAttribute(&managed, hipDeviceAttributeManagedMemory, 0));
  HK(hipDeviceGetAttribute(&concurrent, hipDeviceAttributeConcurrentManagedAccess, 0));
  HK(hipDeviceGetAttribute(&pageable, hipDeviceAttributePageableMemoryAccess, 0));
  HK(hipDeviceGetAttribute(&host_tables, hipDeviceAttributePageableMemoryAccessUsesHostPageTables, 0));
  printf("# MEMORY_CAPS,mapped=%d,managed=%d,concurrent_managed=%d,pageable=%d,host_page_tables=%d,integrated=%d\n",
         p.canMapHostMemory, managed, concurrent, pageable, host_tables, p.integrated);
  if (memory_info) return 0;
  if (((allocation == Alloc::Mapped || allocation == Alloc::Hybrid) && !p.canMapHostMemory) ||
      (allocation == Alloc::Managed && !managed)) {
    fprintf(stderr, "Requested allocator is unsupported on this device\n");
    return 1;
  }
  printf("# %s %s %d CUs, LDS/block %zu, L2 %d MB, B=%d H=%d\n", p.name, p.gcnArchName, p.multiProcessorCount,
         p.sharedMemPerBlock, p.l2CacheSize >> 20, B, H);
  printf("# calibration seed=%llu, input_scale=%.9e, max_error=%.9e, io=%s,allocator=%s,kernel=%s\n",
         (unsigned long long)g_rng, input_scale, max_error, io, alloc_name(allocation),
         kernel_mode == 0 ? "legacy" : kernel_mode == 1 ? "cached" : "auto");
  printf("# RESULT,L,method,config,ms,rel_err\n");
  printf(
      "# MEMORY,L,allocator,owned_bytes,persistent_host_shadow_bytes,allocation_ms,upload_bytes,download_bytes,"
      "copy_ms,setup_ms\n");
  if (max_error > 0) printf("# SELECT,L,method,config,ms,rel_err,max_error,io\n");
  fflush(stdout);
  for (int L = 128; L <= 16384; L *= 2) {
    if (only ? only != L : L > 8192) continue;
    Bench b(L, B, H, input_scale, allocation, concurrent != 0, kernel_mode);
    b.baseline();
    b.variants();
    if (max_error > 0 && !b.select(max_error, io)) failed++;
    b.report_memory();
    fflush(stdout);
  }
  return failed ? 2 : 0;
}
