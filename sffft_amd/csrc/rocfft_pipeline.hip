// rocFFT comparator pipeline (measurement infrastructure, see rocfft_pipeline.h).
#include <hip/hip_runtime.h>
#include <rocfft/rocfft.h>

#include <cstdlib>
#include <mutex>

#include "rocfft_pipeline.h"

struct sffft_rocfft {
  int B, H, L, N, M;
  size_t BH;
  hipStream_t stream;
  float *up, *yp;
  float2 *U, *Kc, *Kh;
  rocfft_plan fwd, inv, kplan;
  rocfft_execution_info info;
  void* work;
};

namespace {

std::once_flag g_setup;

__global__ void pad_kernel(const float* __restrict__ u, float* __restrict__ up, size_t BH, int L) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= BH * 2 * L) return;
  const size_t s = i / (2 * L);
  const int n = (int)(i % (2 * L));
  up[i] = n < L ? u[s * L + n] : 0.f;
}
__global__ void real_to_complex_pad_kernel(const float* __restrict__ k, float2* __restrict__ kc, int H, int L) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)H * 2 * L) return;
  const size_t h = i / (2 * L);
  const int n = (int)(i % (2 * L));
  kc[i] = make_float2(n < L ? k[h * L + n] : 0.f, 0.f);
}
__global__ void half_kernel(const float2* __restrict__ kc, float2* __restrict__ kh, int H, int N) {
  const int M = N / 2 + 1;
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)H * M) return;
  const size_t h = i / M;
  const int k = (int)(i % M);
  const float2 q = kc[h * N + k];
  kh[i] = make_float2(q.x / N, q.y / N);
}
__global__ void mul_kernel(float2* __restrict__ U, const float2* __restrict__ kh, size_t BH, int H, int M) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= BH * M) return;
  const size_t s = i / M;
  const int k = (int)(i % M), h = (int)(s % H);
  const float2 q = kh[(size_t)h * M + k], a = U[i];
  U[i] = make_float2(a.x * q.x - a.y * q.y, a.x * q.y + a.y * q.x);
}
__global__ void slice_kernel(const float* __restrict__ yp, float* __restrict__ y, size_t BH, int L) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= BH * L) return;
  const size_t s = i / L;
  const int n = (int)(i % L);
  y[i] = yp[s * 2 * L + n];
}

unsigned blocks(size_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

extern "C" {

int sffft_rocfft_create(int B, int H, int L, void* stream, sffft_rocfft** out) {
  if (!out || B < 1 || H < 1 || L < 1) return 1;
  std::call_once(g_setup, [] { rocfft_setup(); });
  sffft_rocfft* h = (sffft_rocfft*)calloc(1, sizeof(sffft_rocfft));
  h->B = B; h->H = H; h->L = L; h->N = 2 * L; h->M = L + 1;
  h->BH = (size_t)B * H;
  h->stream = (hipStream_t)stream;
  const size_t len = (size_t)h->N;
  if (hipMalloc(&h->up, h->BH * h->N * 4) || hipMalloc(&h->yp, h->BH * h->N * 4) ||
      hipMalloc(&h->U, h->BH * h->M * 8) || hipMalloc(&h->Kc, (size_t)H * h->N * 8) ||
      hipMalloc(&h->Kh, (size_t)H * h->M * 8)) {
    sffft_rocfft_destroy(h);
    return 3;
  }
  if (rocfft_plan_create(&h->fwd, rocfft_placement_notinplace, rocfft_transform_type_real_forward,
                         rocfft_precision_single, 1, &len, h->BH, nullptr) != rocfft_status_success ||
      rocfft_plan_create(&h->inv, rocfft_placement_notinplace, rocfft_transform_type_real_inverse,
                         rocfft_precision_single, 1, &len, h->BH, nullptr) != rocfft_status_success ||
      rocfft_plan_create(&h->kplan, rocfft_placement_inplace, rocfft_transform_type_complex_forward,
                         rocfft_precision_single, 1, &len, (size_t)H, nullptr) != rocfft_status_success) {
    sffft_rocfft_destroy(h);
    return 4;
  }
  size_t w0 = 0, w1 = 0, w2 = 0;
  rocfft_plan_get_work_buffer_size(h->fwd, &w0);
  rocfft_plan_get_work_buffer_size(h->inv, &w1);
  rocfft_plan_get_work_buffer_size(h->kplan, &w2);
  size_t w = w0 > w1 ? w0 : w1;
  w = w > w2 ? w : w2;
  rocfft_execution_info_create(&h->info);
  if (w) {
    if (hipMalloc(&h->work, w)) {
      sffft_rocfft_destroy(h);
      return 3;
    }
    rocfft_execution_info_set_work_buffer(h->info, h->work, w);
  }
  rocfft_execution_info_set_stream(h->info, h->stream);
  *out = h;
  return 0;
}

int sffft_rocfft_filter(sffft_rocfft* h, const float* k, void* kc) {
  if (!h || !k) return 1;
  hipLaunchKernelGGL(real_to_complex_pad_kernel, dim3(blocks((size_t)h->H * h->N)), dim3(256), 0, h->stream, k,
                     h->Kc, h->H, h->L);
  void* buf[1] = {h->Kc};
  if (rocfft_execute(h->kplan, buf, nullptr, h->info) != rocfft_status_success) return 4;
  hipLaunchKernelGGL(half_kernel, dim3(blocks((size_t)h->H * h->M)), dim3(256), 0, h->stream, h->Kc, h->Kh, h->H,
                     h->N);
  if (kc && hipMemcpyAsync(kc, h->Kc, (size_t)h->H * h->N * 8, hipMemcpyDeviceToDevice, h->stream)) return 3;
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

int sffft_rocfft_core(sffft_rocfft* h) {
  void* in[1] = {h->up};
  void* mid[1] = {h->U};
  void* out[1] = {h->yp};
  if (rocfft_execute(h->fwd, in, mid, h->info) != rocfft_status_success) return 4;
  hipLaunchKernelGGL(mul_kernel, dim3(blocks(h->BH * h->M)), dim3(256), 0, h->stream, h->U, h->Kh, h->BH, h->H,
                     h->M);
  if (rocfft_execute(h->inv, mid, out, h->info) != rocfft_status_success) return 4;
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

int sffft_rocfft_full(sffft_rocfft* h, const float* u, float* y) {
  if (!h || !u || !y) return 1;
  hipLaunchKernelGGL(pad_kernel, dim3(blocks(h->BH * h->N)), dim3(256), 0, h->stream, u, h->up, h->BH, h->L);
  const int rc = sffft_rocfft_core(h);
  if (rc) return rc;
  hipLaunchKernelGGL(slice_kernel, dim3(blocks(h->BH * h->L)), dim3(256), 0, h->stream, h->yp, y, h->BH, h->L);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

void sffft_rocfft_destroy(sffft_rocfft* h) {
  if (!h) return;
  if (h->fwd) rocfft_plan_destroy(h->fwd);
  if (h->inv) rocfft_plan_destroy(h->inv);
  if (h->kplan) rocfft_plan_destroy(h->kplan);
  if (h->info) rocfft_execution_info_destroy(h->info);
  (void)hipFree(h->up);
  (void)hipFree(h->yp);
  (void)hipFree(h->U);
  (void)hipFree(h->Kc);
  (void)hipFree(h->Kh);
  (void)hipFree(h->work);
  free(h);
}

}  // extern "C"
