// Seeded ES generation: the population theta + sigma * [eps; -eps] and the update
// theta + lr * sum_m rank_m eps_m / (P sigma), with eps regenerated from the counter RNG
// (es_noise.h) instead of stored. Replaces the noise lines of the reference's generation
// (es.py:218-226): no (P, D) noise tensor, no (P, D) product in the update.
#include <atomic>
#include <mutex>

#include "es_noise.h"

namespace hipenvs {
namespace esn {

// One thread per (member pair, weight pair): four weights, members m and m + P/2.
// Rows: pairs run fastest within a member, so a wave writes contiguous row segments.
// Columns: members run fastest, so a wave writes 64 consecutive members of one weight row.
template <int kLayout>
__global__ __launch_bounds__(kBlock) void perturb_kernel(const float* __restrict__ theta, int64_t d, int64_t p,
                                                         uint32_t seed, float sigma, uint32_t pairs,
                                                         uint32_t half, float* __restrict__ out) {
  const uint64_t idx = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  if (idx >= (uint64_t)pairs * half) return;
  uint32_t m, j;
  if (kLayout == kPerturbRows) {
    m = (uint32_t)(idx / pairs);
    j = (uint32_t)(idx - (uint64_t)m * pairs);
  } else {
    j = (uint32_t)(idx / half);
    m = (uint32_t)(idx - (uint64_t)j * half);
  }
  float z0, z1;
  gauss_pair(member_key(seed, m), j, z0, z1);
  const int64_t k = 2 * (int64_t)j;
  const float e0 = sigma * z0, e1 = sigma * z1;
  const int64_t ma = m, mb = (int64_t)m + half;
  const float t0 = theta[k];
  if (kLayout == kPerturbRows) {
    out[ma * d + k] = t0 + e0;
    out[mb * d + k] = t0 + -e0;
    if (k + 1 < d) {
      const float t1 = theta[k + 1];
      out[ma * d + k + 1] = t1 + e1;
      out[mb * d + k + 1] = t1 + -e1;
    }
  } else {
    out[k * p + ma] = t0 + e0;
    out[k * p + mb] = t0 + -e0;
    if (k + 1 < d) {
      const float t1 = theta[k + 1];
      out[(k + 1) * p + ma] = t1 + e1;
      out[(k + 1) * p + mb] = t1 + -e1;
    }
  }
}

// Partial sums of the update: block (x, c) covers weight pairs 64x .. 64x + 63 (one per lane)
// and member pairs [c * mc, (c + 1) * mc); each lane sums w_m * eps_m[2j], w_m * eps_m[2j + 1]
// over its chunk in member order, with w_m = rank_m - rank_{m + P/2}. The member key and
// weight are the same for the whole wave.
__global__ __launch_bounds__(64) void noise_partial_kernel(const float* __restrict__ ranks, int64_t d,
                                                           uint32_t half, uint32_t pairs, uint32_t seed,
                                                           uint32_t mc, float* __restrict__ partial) {
  const uint32_t j = blockIdx.x * 64u + threadIdx.x;
  const uint32_t c = blockIdx.y;
  const uint32_t m0 = c * mc, m1 = m0 + mc < half ? m0 + mc : half;
  float acc0 = 0.0f, acc1 = 0.0f;
  for (uint32_t m = m0; m < m1; ++m) {
    const float w = ranks[m] - ranks[m + half];
    float z0, z1;
    gauss_pair(member_key(seed, m), j, z0, z1);
    acc0 = acc0 + w * z0;
    acc1 = acc1 + w * z1;
  }
  if (j >= pairs) return;
  const int64_t k = 2 * (int64_t)j;
  partial[(int64_t)c * d + k] = acc0;
  if (k + 1 < d) partial[(int64_t)c * d + k + 1] = acc1;
}

// theta + lr * (sum over chunks, in chunk order) / scale. out may alias theta: each thread
// reads theta[k] and then writes out[k].
__global__ __launch_bounds__(kBlock) void update_kernel(const float* theta, const float* __restrict__ partial,
                                                        int64_t d, uint32_t chunks, float scale, float lr,
                                                        float* out) {
  const int64_t k = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (k >= d) return;
  float total = 0.0f;
  for (uint32_t c = 0; c < chunks; ++c) total = total + partial[(int64_t)c * d + k];
  out[k] = theta[k] + lr * (total / scale);
}

inline int64_t update_chunks(int64_t half) { return (half + chunk_members(half) - 1) / chunk_members(half); }

}  // namespace esn

int launch_perturb(const float* theta, int64_t d, int64_t p, uint32_t seed, float sigma, int layout, float* out,
                   hipStream_t s) {
  const uint32_t half = (uint32_t)(p / 2), pairs = (uint32_t)((d + 1) / 2);
  const uint64_t items = (uint64_t)half * pairs;
  const dim3 grid((unsigned)((items + kBlock - 1) / kBlock)), block(kBlock);
  if (layout == kPerturbRows)
    hipLaunchKernelGGL(esn::perturb_kernel<kPerturbRows>, grid, block, 0, s, theta, d, p, seed, sigma, pairs, half,
                       out);
  else
    hipLaunchKernelGGL(esn::perturb_kernel<kPerturbColumns>, grid, block, 0, s, theta, d, p, seed, sigma, pairs,
                       half, out);
  return launch_status();
}

}  // namespace hipenvs

using namespace hipenvs;

namespace {
// p even and at least 2, d >= 1, and every index of the kernels inside 32-bit member and
// pair counts and a 2^32 - 1 block grid.
bool population_ok(int64_t d, int64_t p) {
  if (d < 1 || p < 2 || (p & 1) || p > 0x7fffffffLL || d > 0x7fffffffLL) return false;
  const uint64_t items = (uint64_t)(p / 2) * (uint64_t)((d + 1) / 2);
  return items / kBlock < 0xffffffffULL;
}
}  // namespace

extern "C" int hipenvs_es_perturb(const float* theta, int64_t d, int64_t p, uint32_t seed, double sigma,
                                  int32_t layout, float* out, hipenvs_stream_t stream) {
  if (!population_ok(d, p) || (layout != 0 && layout != 1) || !theta || !out) return HIPENVS_E_ARG;
  return launch_perturb(theta, d, p, seed, (float)sigma, layout, out, as_stream(stream));
}

extern "C" int64_t hipenvs_es_update_workspace_bytes(int64_t d, int64_t p) {
  if (!population_ok(d, p)) return -1;
  return (int64_t)sizeof(float) * esn::update_chunks(p / 2) * d;
}

namespace {
// The update's two launches with its partial sums in `partial` (update_chunks(p / 2) x d floats).
int launch_update(const float* theta, const float* ranks, int64_t d, int64_t p, uint32_t seed, double sigma,
                  double lr, float* theta_out, float* partial, hipStream_t s) {
  const int64_t half = p / 2, mc = esn::chunk_members(half), chunks = esn::update_chunks(half);
  const uint32_t pairs = (uint32_t)((d + 1) / 2);
  hipLaunchKernelGGL(esn::noise_partial_kernel, dim3((pairs + 63) / 64, (unsigned)chunks), dim3(64), 0, s, ranks, d,
                     (uint32_t)half, pairs, seed, (uint32_t)mc, partial);
  int status = launch_status();
  if (status != HIPENVS_OK) return status;
  // the caller's P * sigma in double (es.py:224), rounded once to float32 as numpy does for a Python scalar
  const float scale = (float)((double)p * sigma);
  hipLaunchKernelGGL(esn::update_kernel, dim3(grid_for(d)), dim3(kBlock), 0, s, theta, partial, d, (uint32_t)chunks,
                     scale, (float)lr, theta_out);
  return launch_status();
}

// Static partial-sum buffer of hipenvs_es_update_static: each GPU the library runs on holds
// its own copy until the process ends. Host code never uses the array's name as an address
// (on the host it is only a stand-in for the device symbol); it uses the device address that
// hipGetSymbolAddress returns, looked up once per device with that device current.
constexpr int64_t kStaticPartialFloats = HIPENVS_ES_UPDATE_STATIC_BYTES / (int64_t)sizeof(float);
__device__ __align__(256) float scratch[kStaticPartialFloats];

std::atomic<float*> g_scratch[kMaxDevices];
std::mutex g_scratch_mutex;

// The current device's address of `scratch`, or a negative status.
int static_partials(float** out) {
  int dev = 0;
  const int status = current_device(&dev);
  if (status != HIPENVS_OK) return status;
  hipError_t e = hipSuccess;
  float* ptr = g_scratch[dev].load(std::memory_order_acquire);
  if (!ptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    ptr = g_scratch[dev].load(std::memory_order_relaxed);
    if (!ptr) {
      void* addr = nullptr;
      e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !addr) {
        set_last_hip_error((int)(e != hipSuccess ? e : hipErrorInvalidSymbol));
        return HIPENVS_E_HIP;
      }
      ptr = static_cast<float*>(addr);
      g_scratch[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return HIPENVS_OK;
}
}  // namespace

extern "C" int hipenvs_es_update(const float* theta, const float* ranks, int64_t d, int64_t p, uint32_t seed,
                                 double sigma, double lr, float* theta_out, void* workspace,
                                 int64_t workspace_bytes, hipenvs_stream_t stream) {
  if (!population_ok(d, p) || !theta || !ranks || !theta_out || !workspace) return HIPENVS_E_ARG;
  if (workspace_bytes < hipenvs_es_update_workspace_bytes(d, p)) return HIPENVS_E_ARG;
  return launch_update(theta, ranks, d, p, seed, sigma, lr, theta_out, static_cast<float*>(workspace),
                       as_stream(stream));
}

extern "C" int hipenvs_es_update_static(const float* theta, const float* ranks, int64_t d, int64_t p, uint32_t seed,
                                        double sigma, double lr, float* theta_out, hipenvs_stream_t stream) {
  if (!population_ok(d, p) || !theta || !ranks || !theta_out) return HIPENVS_E_ARG;
  if (hipenvs_es_update_workspace_bytes(d, p) > HIPENVS_ES_UPDATE_STATIC_BYTES) return HIPENVS_E_SCRATCH;
  float* partial = nullptr;
  const int status = static_partials(&partial);
  if (status != HIPENVS_OK) return status;
  // every partial the update kernel reads is written first by the partial kernel of the same
  // call, so nothing is cleared
  return launch_update(theta, ranks, d, p, seed, sigma, lr, theta_out, partial, as_stream(stream));
}
