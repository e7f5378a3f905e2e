/*
 * mojogp_amd — C ABI of the MI355X (gfx950) exact-GP engine.
 *
 * Drop-in boundary for the reference's two native modules (caspbian/mojogp):
 *   - the generated kernel module (init_provider / materialize /
 *     destroy_provider and the fn-pointer table it returns),
 *     mojogp/codegen_engine/emit/fn_ptr_module.py:998-1211, 1120-1166;
 *   - the engine module (train / predict / prediction cache /
 *     benchmark_provider_ops), mojogp/kernels/jit/jit_engine_bindings.mojo:1750-1775.
 *
 * Conventions
 *   - Every function returns 0 on success or a non-zero status; the message is
 *     available from mgp_last_error() (per thread).
 *   - Arrays are host pointers unless the name ends in _device.  Matrices of
 *     right-hand sides are column-major [ncols][n] (element c*n + i), as in the
 *     reference (fn_ptr_module.py:391-491).  Inputs X are row-major [n][d].
 *   - Every call is synchronous on return.  Each provider owns one HIP stream;
 *     a handle must not be used from two threads at once.
 *   - Kernel kinds: 0 = RBF, 1 = Matern-5/2.  Parameter layout (engine layout,
 *     mojogp/kernel.py:494-509): isotropic [lengthscale, outputscale];
 *     ARD [ls_0 .. ls_{d-1}, outputscale].
 */
#ifndef MOJOGP_AMD_H
#define MOJOGP_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MGP_API __attribute__((visibility("default")))

/* Status codes. */
#define MGP_OK 0
#define MGP_ERR_INVALID 1
#define MGP_ERR_HIP 2
#define MGP_ERR_NUMERIC 3
#define MGP_ERR_INTERNAL 4

/* Copies the calling thread's last error message into buf (NUL terminated,
 * truncated to len-1 bytes); returns the full message length.
 * Replaces the Python exceptions raised by the reference's `raises` functions
 * (jit_engine_bindings.mojo:163-164, 479-480). */
MGP_API int mgp_last_error(char* buf, size_t len);
MGP_API const char* mgp_version(void);
MGP_API int mgp_device_count(int* out);

/* ---- Provider (kernel module) ------------------------------------------ */

/* Creates a device-resident provider for training inputs X[n][d].
 * Replaces init_provider(X, params, noise) (fn_ptr_module.py:998-1168). */
MGP_API int mgp_init_provider(int kind, int ard, int d, int64_t n,
                              const float* X, const float* params, int nparams,
                              float noise, void** out_handle);
/* Replaces destroy_provider(info) (fn_ptr_module.py:1183-1195). */
MGP_API int mgp_destroy_provider(void* handle);
/* Replace the impl_update_params / impl_update_noise / impl_get_noise /
 * impl_get_diagonal_value fn pointers (fn_ptr_module.py:651-703). */
MGP_API int mgp_update_params(void* handle, const float* params, int nparams);
MGP_API int mgp_update_noise(void* handle, float noise);
MGP_API int mgp_get_noise(void* handle, float* out);
MGP_API int mgp_get_diagonal_value(void* handle, float* out);
/* Shape of a provider (the n / dim / num_gradient_params / is_ard keys of the
 * reference's provider dict, fn_ptr_module.py:1120-1166). */
MGP_API int mgp_provider_info(void* handle, int64_t* n, int* d, int* nparams,
                              int* kind, int* ard);

/* out = (K + noise I) V.  Replaces the forward_matvec fn pointer
 * (impl_forward_matvec, fn_ptr_module.py:391-491). */
MGP_API int mgp_forward_matvec(void* handle, const float* V, int ncols,
                               float* out);
/* Same with device-resident V/out (no PCIe copies). */
MGP_API int mgp_forward_matvec_device(void* handle, const float* V_device,
                                      int ncols, float* out_device);
/* (K + noise I) V from per-dimension differences (no Gram form, no MFMA):
 * an independent device cross-check of mgp_forward_matvec.  No reference
 * counterpart; kept for parity tests. */
MGP_API int mgp_direct_matvec(void* handle, const float* V, int ncols,
                              float* out);
/* out[c*m + i] = sum_j k(Xs_i, X_j) V[c*n + j].  Replaces the cross_matvec fn
 * pointer (impl_cross_matvec, fn_ptr_module.py:576-626). */
MGP_API int mgp_cross_matvec(void* handle, const float* Xs, int64_t m,
                             const float* V, int ncols, float* out);
/* diag k(x_i, x_i).  Replace extract_diagonal / extract_diagonal_test
 * (fn_ptr_module.py:628-649). */
MGP_API int mgp_extract_diagonal(void* handle, float* out);
MGP_API int mgp_extract_diagonal_test(void* handle, const float* Xs, int64_t m,
                                      float* out);

/* Isolated timing of provider ops.  Replaces benchmark_provider_ops(info, rhs,
 * num_cols, op_code, repeats, warmup) (jit_engine_bindings.mojo:439-572);
 * op 0 = forward matvec.  times_ms[repeats] gets per-call host wall times,
 * tile_ms_avg the mean HIP-event duration of the fused tile kernel, and
 * out_or_null (if non-null) the last output. */
MGP_API int mgp_benchmark_provider_ops(void* handle, const float* rhs,
                                       int ncols, int op, int repeats,
                                       int warmup, double* times_ms,
                                       double* tile_ms_avg, float* out_or_null);

/* Streaming device copy of `bytes` repeated `repeats` times; ms_avg gets the
 * mean duration of one copy.  Used only to calibrate HBM byte counters
 * (FETCH_SIZE / WRITE_SIZE) against a kernel of known traffic.  No reference
 * counterpart. */
MGP_API int mgp_calibration_copy(int64_t bytes, int repeats, double* ms_avg);

#ifdef __cplusplus
}
#endif

#endif /* MOJOGP_AMD_H */
