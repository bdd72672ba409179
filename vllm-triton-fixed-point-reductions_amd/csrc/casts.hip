// Elementwise float <-> fixed-point casts (HBM streaming kernels).
//
// Replaces fxpr_vllm/_triton/casts.py:21-54 (_float_to_fixed_kernel,
// _fixed_to_float_kernel). Each thread moves one 16-byte vector of the input;
// a scalar variant covers misaligned views.

#include "fxp_device.h"
#include "fxpr_internal.h"

namespace fxpr {
namespace {

constexpr int kThreads = 256;

template <typename T, int N> struct alignas(sizeof(T) * N) Vec { T v[N]; };

template <int XDT> struct FloatIn;
template <> struct FloatIn<FXPR_DTYPE_F16> { using T = uint16_t; static __device__ float get(T v) { return f16_to_f32(v); } };
template <> struct FloatIn<FXPR_DTYPE_F32> { using T = float;    static __device__ float get(T v) { return v; } };
template <> struct FloatIn<FXPR_DTYPE_F64> { using T = double;   static __device__ float get(T v) { return static_cast<float>(v); } };

template <int BITS> struct IntOf;
template <> struct IntOf<16> { using T = int16_t; };
template <> struct IntOf<32> { using T = int32_t; };
template <> struct IntOf<64> { using T = int64_t; };

// q = RNE_sat_BITS(fl32(x) * 2^f)
template <int XDT, int BITS, int VEC>
__global__ __launch_bounds__(kThreads) void float_to_fixed_kernel(
    const typename FloatIn<XDT>::T* __restrict__ x, typename IntOf<BITS>::T* __restrict__ q,
    int64_t n, float scale) {
  using XT = typename FloatIn<XDT>::T;
  using QT = typename IntOf<BITS>::T;
  const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * VEC;
  if (i0 >= n) return;
  if (VEC > 1 && i0 + VEC <= n) {
    Vec<XT, VEC> xv = *reinterpret_cast<const Vec<XT, VEC>*>(x + i0);
    Vec<QT, VEC> qv;
#pragma unroll
    for (int j = 0; j < VEC; ++j)
      qv.v[j] = static_cast<QT>(quant<BITS>(__fmul_rn(FloatIn<XDT>::get(xv.v[j]), scale)));
    *reinterpret_cast<Vec<QT, VEC>*>(q + i0) = qv;
  } else {
    for (int64_t i = i0; i < n && i < i0 + VEC; ++i)
      q[i] = static_cast<QT>(quant<BITS>(__fmul_rn(FloatIn<XDT>::get(x[i]), scale)));
  }
}

template <int FBITS> struct FloatOut;
template <> struct FloatOut<16> { using T = uint16_t; static __device__ T put(float f) { return f32_to_f16(f); } };
template <> struct FloatOut<32> { using T = float;    static __device__ T put(float f) { return f; } };
template <> struct FloatOut<64> { using T = double;   static __device__ T put(float f) { return static_cast<double>(f); } };

template <int QBITS, typename QT> __device__ __forceinline__ float to_f32(QT v, float inv) {
  if constexpr (QBITS <= 32) return fixed_to_f32(static_cast<int32_t>(v), inv);
  else return fixed_to_f32(static_cast<int64_t>(v), inv);
}

// y = OUT(fl32(q) * 2^-f)
template <int QBITS, int FBITS, int VEC>
__global__ __launch_bounds__(kThreads) void fixed_to_float_kernel(
    const typename IntOf<QBITS>::T* __restrict__ q, typename FloatOut<FBITS>::T* __restrict__ y,
    int64_t n, float inv_scale) {
  using QT = typename IntOf<QBITS>::T;
  using YT = typename FloatOut<FBITS>::T;
  const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * VEC;
  if (i0 >= n) return;
  if (VEC > 1 && i0 + VEC <= n) {
    Vec<QT, VEC> qv = *reinterpret_cast<const Vec<QT, VEC>*>(q + i0);
    Vec<YT, VEC> yv;
#pragma unroll
    for (int j = 0; j < VEC; ++j)
      yv.v[j] = FloatOut<FBITS>::put(to_f32<QBITS>(qv.v[j], inv_scale));
    *reinterpret_cast<Vec<YT, VEC>*>(y + i0) = yv;
  } else {
    for (int64_t i = i0; i < n && i < i0 + VEC; ++i)
      y[i] = FloatOut<FBITS>::put(to_f32<QBITS>(q[i], inv_scale));
  }
}

template <int XDT, int BITS>
int launch_f2q(const void* x, void* q, int64_t n, float scale, hipStream_t st) {
  using XT = typename FloatIn<XDT>::T;
  using QT = typename IntOf<BITS>::T;
  constexpr int VEC = 16 / sizeof(XT);
  if (aligned(x, 16) && aligned(q, sizeof(QT) * VEC)) {
    dim3 grid(static_cast<unsigned>(cdiv(n, int64_t(kThreads) * VEC)));
    float_to_fixed_kernel<XDT, BITS, VEC><<<grid, kThreads, 0, st>>>(
        static_cast<const XT*>(x), static_cast<QT*>(q), n, scale);
  } else {
    dim3 grid(static_cast<unsigned>(cdiv(n, kThreads)));
    float_to_fixed_kernel<XDT, BITS, 1><<<grid, kThreads, 0, st>>>(
        static_cast<const XT*>(x), static_cast<QT*>(q), n, scale);
  }
  return launch_status();
}

template <int QBITS, int FBITS>
int launch_q2f(const void* q, void* y, int64_t n, float inv_scale, hipStream_t st) {
  using QT = typename IntOf<QBITS>::T;
  using YT = typename FloatOut<FBITS>::T;
  constexpr int VEC = 16 / sizeof(QT) < 2 ? 2 : 16 / sizeof(QT);
  if (aligned(q, sizeof(QT) * VEC) && aligned(y, sizeof(YT) * VEC)) {
    dim3 grid(static_cast<unsigned>(cdiv(n, int64_t(kThreads) * VEC)));
    fixed_to_float_kernel<QBITS, FBITS, VEC><<<grid, kThreads, 0, st>>>(
        static_cast<const QT*>(q), static_cast<YT*>(y), n, inv_scale);
  } else {
    dim3 grid(static_cast<unsigned>(cdiv(n, kThreads)));
    fixed_to_float_kernel<QBITS, FBITS, 1><<<grid, kThreads, 0, st>>>(
        static_cast<const QT*>(q), static_cast<YT*>(y), n, inv_scale);
  }
  return launch_status();
}

template <int XDT>
int dispatch_f2q_bits(const void* x, void* q, int bits, int64_t n, float scale, hipStream_t st) {
  switch (bits) {
    case 16: return launch_f2q<XDT, 16>(x, q, n, scale, st);
    case 32: return launch_f2q<XDT, 32>(x, q, n, scale, st);
    default: return launch_f2q<XDT, 64>(x, q, n, scale, st);
  }
}

template <int QBITS>
int dispatch_q2f_bits(const void* q, void* y, int fbits, int64_t n, float inv, hipStream_t st) {
  switch (fbits) {
    case 16: return launch_q2f<QBITS, 16>(q, y, n, inv, st);
    case 32: return launch_q2f<QBITS, 32>(q, y, n, inv, st);
    default: return launch_q2f<QBITS, 64>(q, y, n, inv, st);
  }
}

}  // namespace
}  // namespace fxpr

using namespace fxpr;

// The scale 2^f is exact in fp32 for every f the ABI accepts (0..63), and so
// is 2^-f, matching fxp_constants (fxpr_vllm/_triton/fxp.py:40-41).
extern "C" int fxpr_float_to_fixed(const void* x, int x_dtype, void* q, int int_bits,
                                   int frac_bits, int64_t n, void* stream) {
  if (!valid_int_bits(int_bits) || frac_bits < 0 || frac_bits > 63) return FXPR_E_BITS;
  if (n < 0) return FXPR_E_SHAPE;
  if (n == 0) return FXPR_OK;
  if (!x || !q) return FXPR_E_ARG;
  const float scale = pow2f(frac_bits);
  hipStream_t st = as_stream(stream);
  switch (x_dtype) {
    case FXPR_DTYPE_F16: return dispatch_f2q_bits<FXPR_DTYPE_F16>(x, q, int_bits, n, scale, st);
    case FXPR_DTYPE_F32: return dispatch_f2q_bits<FXPR_DTYPE_F32>(x, q, int_bits, n, scale, st);
    case FXPR_DTYPE_F64: return dispatch_f2q_bits<FXPR_DTYPE_F64>(x, q, int_bits, n, scale, st);
    default: return FXPR_E_DTYPE;
  }
}

extern "C" int fxpr_fixed_to_float(const void* q, int q_dtype, void* y, int float_bits,
                                   int frac_bits, int64_t n, void* stream) {
  if (!(float_bits == 16 || float_bits == 32 || float_bits == 64)) return FXPR_E_BITS;
  if (frac_bits < 0 || frac_bits > 63) return FXPR_E_BITS;
  if (n < 0) return FXPR_E_SHAPE;
  if (n == 0) return FXPR_OK;
  if (!q || !y) return FXPR_E_ARG;
  const float inv = pow2f(-frac_bits);
  hipStream_t st = as_stream(stream);
  switch (q_dtype) {
    case FXPR_DTYPE_I16: return dispatch_q2f_bits<16>(q, y, float_bits, n, inv, st);
    case FXPR_DTYPE_I32: return dispatch_q2f_bits<32>(q, y, float_bits, n, inv, st);
    case FXPR_DTYPE_I64: return dispatch_q2f_bits<64>(q, y, float_bits, n, inv, st);
    default: return FXPR_E_DTYPE;
  }
}

extern "C" int fxpr_abi_version(void) { return 3; }

extern "C" const char* fxpr_error_string(int code) {
  switch (code) {
    case FXPR_OK: return "success";
    case FXPR_E_DTYPE: return "fxpr: unsupported element type";
    case FXPR_E_BITS: return "fxpr: int_bits / frac_bits / float_bits out of range";
    case FXPR_E_SHAPE: return "fxpr: invalid or inconsistent sizes";
    case FXPR_E_WORKSPACE: return "fxpr: workspace missing or too small";
    case FXPR_E_ARG: return "fxpr: invalid argument";
    case FXPR_E_CAPTURE:
      return "fxpr: first use on this device while the stream is capturing a graph (make one eager call first)";
    default:
      if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
      return "fxpr: unknown error";
  }
}
