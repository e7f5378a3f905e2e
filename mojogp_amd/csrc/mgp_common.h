// Shared definitions for the MI355X (gfx950) exact-GP engine.
//
// Every exported entry point returns an int status (0 = OK) and records a
// human-readable message retrievable with mgp_last_error().  Device errors are
// converted to status codes at the boundary; nothing throws across the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

namespace mgp {

// Kernel families handled by the hand-written kernels.  Values are part of the
// C ABI (include/mojogp_amd.h).
enum KernelKind : int { KIND_RBF = 0, KIND_MATERN52 = 1, KIND_MATERN12 = 2, KIND_MATERN32 = 3 };
inline bool valid_kind(int kind) { return kind >= KIND_RBF && kind <= KIND_MATERN32; }

// ln(2) and log2(e) in float.
constexpr float kLn2 = 0.69314718055994530942f;
constexpr float kLog2e = 1.44269504088896340736f;
// exp(max(x, -20)) clamp of the reference's numerical-stability pass, expressed
// in base 2: 20 * log2(e).
constexpr float kExp2Clamp = 20.0f * 1.44269504088896340736f;
// Exponent limit standing for "no clamp" (exp2 of anything beyond it is 0).
constexpr float kExp2NoClamp = 3.0e38f;

// Where the reference's generated code clamps a leaf's exponent.  Its
// numerical-stability pass rewrites exp(x) as exp(max(x, -20)) only when x is
// syntactically a negative constant, a product with a negative constant as a
// direct operand, or c - y with c <= 0 (passes/numerical_stability.py:29-41,
// 62-85), after products were left-nested (ir.py:183-190) and CSE ran.  The
// emitted expressions (recorded per kind, iso/ARD and d in
// tests/golden/ref_kernel_exprs.json) therefore clamp
//   Matern-3/2, Matern-5/2 (iso and ARD):  exp(max(-1 * u, -20)),
//   Matern-1/2 ARD:                         exp(max(-1 * r, -20)),
// and leave unclamped
//   RBF (iso: exp((-0.5 dist_sq) inv_l^2); ARD: exp(sum of per-dimension terms)),
//   Matern-1/2 isotropic (exp((-1 r_raw) inv_l)), periodic leaves.
// The limit on the base-2 exponent (u or s) of one leaf:
inline float exp2_limit(int kind, bool ard) {
  if (kind == KIND_RBF) return kExp2NoClamp;
  if (kind == KIND_MATERN12 && !ard) return kExp2NoClamp;
  return kExp2Clamp;
}
// The reference's r = sqrt(r^2 + 1e-20) floor of the Matern-1/2 distance in
// the base-2 scaled coordinates (log2(e)^2 * 1e-20); only the gradient weight
// 1/r needs it.
constexpr float kM12RFloor = 2.0813689810056076e-20f;

// Error carried to the C boundary.
struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

enum Status : int {
  ST_OK = 0,
  ST_INVALID = 1,
  ST_HIP = 2,
  ST_NUMERIC = 3,
  ST_INTERNAL = 4,
};

void set_last_error(const std::string& msg);

#define MGP_HIP_CHECK(expr)                                                    \
  do {                                                                         \
    hipError_t _e = (expr);                                                    \
    if (_e != hipSuccess) {                                                    \
      throw ::mgp::Error(::mgp::ST_HIP,                                   \
                         std::string(#expr) + " failed: " +                    \
                             hipGetErrorString(_e) + " (" __FILE__ ":" +       \
                             std::to_string(__LINE__) + ")");                  \
    }                                                                          \
  } while (0)

#define MGP_REQUIRE(cond, msg)                                                 \
  do {                                                                         \
    if (!(cond)) throw ::mgp::Error(::mgp::ST_INVALID, (msg));            \
  } while (0)

// Wrap the body of an exported function: converts exceptions to status codes.
template <class F>
int guarded(F&& f) {
  try {
    f();
    return ST_OK;
  } catch (const Error& e) {
    set_last_error(e.what());
    return e.code;
  } catch (const std::exception& e) {
    set_last_error(e.what());
    return ST_INTERNAL;
  } catch (...) {
    set_last_error("unknown native error");
    return ST_INTERNAL;
  }
}

// Owning device buffer (hipMalloc'd), grown on demand.
template <class T>
struct DevBuf {
  T* ptr = nullptr;
  size_t count = 0;
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  ~DevBuf() { release(); }
  void release() {
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    count = 0;
  }
  // Ensure capacity for n elements; contents are not preserved on growth.
  T* ensure(size_t n) {
    if (n == 0) n = 1;
    if (n > count) {
      release();
      MGP_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&ptr), n * sizeof(T)));
      count = n;
    }
    return ptr;
  }
};

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

}  // namespace mgp
