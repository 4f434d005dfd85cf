// hip_ops.cpp -- the reference runtime's backend interface (woodcock::ops,
// include/woodcock/ops.h:9-24 of the reference) on this library, the slot next
// to src/backends/cpu_ops.cpp: the runtime's Drafter::forward
// (src/core/drafter.cpp:106-133) and Qwen3::forward (src/core/qwen3.cpp:86-111)
// build against it unchanged.
//
// The reference runtime keeps activations, caches and fp32 weights in host
// memory (std::vector), so each call stages its operands in device memory,
// runs the library's stream-ordered operation (wc_linear, wc_rmsnorm, wc_rope,
// wc_silu_mul, wc_attention, wc_softmax) on the null stream and copies the
// result back.  Nothing is cached between calls: a host buffer's address says
// nothing about whether its contents changed.  This makes the slot a
// correctness path for that runtime, not a fast one -- the fused entry points
// (wc_drafter_forward, wc_draft_head_norm, wc_verify_*) are the fast path.
// Errors from the library or the HIP runtime throw std::runtime_error, as the
// runtime's own code does.
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <mutex>
#include <stdexcept>
#include <string>

#include "woodcock/ops.h"
#include "woodcock_hip.h"

namespace woodcock::ops {
namespace {

void check(int status, const char* what) {
  if (status != WC_OK) throw std::runtime_error(std::string(what) + ": " + wc_last_error());
}
void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// growable device buffers, one per operand slot of a call
struct Slot {
  void* p = nullptr;
  size_t bytes = 0;
  void* get(size_t n) {
    if (n > bytes) {
      if (p) hip_check(hipFree(p), "hipFree");
      p = nullptr;
      bytes = 0;
      hip_check(hipMalloc(&p, n), "hipMalloc");
      bytes = n;
    }
    return p;
  }
};
std::mutex g_mu;
Slot g_slot[6];

template <typename T>
T* put(int slot, const T* host, size_t count) {
  void* d = g_slot[slot].get(count * sizeof(T));
  if (count) hip_check(hipMemcpy(d, host, count * sizeof(T), hipMemcpyHostToDevice), "copy to device");
  return static_cast<T*>(d);
}
template <typename T>
T* scratch(int slot, size_t count) {
  return static_cast<T*>(g_slot[slot].get(count * sizeof(T)));
}
template <typename T>
void get(T* host, const T* dev, size_t count) {
  // the null stream: ordered after the operation that wrote `dev`
  if (count) hip_check(hipMemcpy(host, dev, count * sizeof(T), hipMemcpyDeviceToHost), "copy to host");
}

}  // namespace

void linear(const float* x, int L, int in, const Tensor& W, float* y, bool accumulate) {
  if (W.cols() != in) throw std::runtime_error("linear: weight columns != input width");
  const int out = static_cast<int>(W.rows());
  std::lock_guard<std::mutex> lk(g_mu);
  const float* dx = put(0, x, size_t(L) * in);
  const float* dw = put(1, W.data.data(), size_t(out) * in);
  float* dy = accumulate ? put(2, y, size_t(L) * out) : scratch<float>(2, size_t(L) * out);
  check(wc_linear(dx, L, in, dw, WC_F32, out, dy, accumulate ? 1 : 0, nullptr), "wc_linear");
  get(y, dy, size_t(L) * out);
}

void rmsnorm(const float* x, float* y, int rows, int d, const float* w, float eps) {
  std::lock_guard<std::mutex> lk(g_mu);
  const float* dx = put(0, x, size_t(rows) * d);
  const float* dw = put(1, w, size_t(d));
  float* dy = scratch<float>(2, size_t(rows) * d);
  check(wc_rmsnorm(dx, dy, rows, d, dw, WC_F32, eps, nullptr), "wc_rmsnorm");
  get(y, dy, size_t(rows) * d);
}

void rope(float* x, int L, int heads, int D, const int* positions, float base) {
  std::lock_guard<std::mutex> lk(g_mu);
  float* dx = put(0, x, size_t(L) * heads * D);
  const int32_t* dp = put(1, reinterpret_cast<const int32_t*>(positions), size_t(L));
  check(wc_rope(dx, L, heads, D, dp, base, nullptr, nullptr, 0, nullptr), "wc_rope");
  get(x, dx, size_t(L) * heads * D);
}

void silu_mul(float* gate, const float* up, int64_t n) {
  std::lock_guard<std::mutex> lk(g_mu);
  float* dg = put(0, gate, size_t(n));
  const float* du = put(1, up, size_t(n));
  check(wc_silu_mul(dg, du, n, nullptr), "wc_silu_mul");
  get(gate, dg, size_t(n));
}

void attention(const float* q, int L, int H, int Hk, int D, const float* K, const float* V, int T,
               const uint8_t* mask, float* out, float scale) {
  std::lock_guard<std::mutex> lk(g_mu);
  const float* dq = put(0, q, size_t(L) * H * D);
  const float* dk = put(1, K, size_t(T) * Hk * D);
  const float* dv = put(2, V, size_t(T) * Hk * D);
  const uint8_t* dm = mask ? put(3, mask, size_t(L) * T) : nullptr;
  float* dout = scratch<float>(4, size_t(L) * H * D);
  check(wc_attention(dq, L, H, Hk, D, dk, dv, T, dm, dout, scale, nullptr), "wc_attention");
  get(out, dout, size_t(L) * H * D);
}

void softmax(float* x, int n) {
  std::lock_guard<std::mutex> lk(g_mu);
  float* dx = put(0, x, size_t(n));
  check(wc_softmax(dx, 1, n, nullptr), "wc_softmax");
  get(x, dx, size_t(n));
}

}  // namespace woodcock::ops
