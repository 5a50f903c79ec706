// RMSNorm (with an optional residual add) and SwiGLU for gfx950: the two elementwise /
// row-reduction ops around the W4A16 linears of a quantized decoder layer.
//
// Semantics follow the reference's eager default paths, rounding for rounding:
//   RMSNorm (slipstream/models/layers/rmsnorm.py:30-33, fused_rmsnorm.py:73-82):
//     s = x + residual            (in the tensor dtype: fp32 sum rounded)
//     x_hat = s * rsqrt(mean(s^2) + eps)   in fp32, rounded to the dtype
//     y = weight * x_hat          (fp32 product rounded to the dtype)
//   SwiGLU (slipstream/models/layers/mlp.py:37-40, fused_swiglu.py:49-50):
//     y = silu(gate) * up         (silu in fp32 rounded to the dtype, then the product)
// Differences from the reference can only come from the fp32 sum order of mean(s^2)
// and from rsqrt/exp, whose last fp32 bits may differ; after rounding to bf16/fp16
// that is at most one unit in the last place, rarely.
//
// Work layout: RMSNorm takes one workgroup per row; each thread holds its 16-byte
// pieces of the row in registers between the reduction and the write (rows up to
// 256 * PPT pieces), so the row is read once. SwiGLU is a grid-stride loop over
// 16-byte pieces.
#include "ss_common.h"

namespace {

template <typename T>
struct Rnd;
template <>
struct Rnd<ss::bf16_t> {
  static __device__ __forceinline__ float r(float x) { return (float)(ss::bf16_t)x; }
};
template <>
struct Rnd<ss::f16_t> {
  static __device__ __forceinline__ float r(float x) { return (float)(ss::f16_t)x; }
};
template <>
struct Rnd<float> {
  static __device__ __forceinline__ float r(float x) { return x; }
};

// keeps an fp32 value from being fused into a following operation (fp-contract) or
// narrowed to 16-bit arithmetic, which would skip one of the reference's roundings
__device__ __forceinline__ float pin(float x) {
  asm volatile("" : "+v"(x));
  return x;
}


template <typename T>
__device__ __forceinline__ void unpack(const ss::u32x4& w, float (&f)[16 / sizeof(T)]) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t u = w[e];
      f[e] = __builtin_bit_cast(float, u);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t u = w[e >> 1];
      const uint16_t h = (uint16_t)((e & 1) ? (u >> 16) : (u & 0xFFFFu));
      f[e] = (float)__builtin_bit_cast(T, h);
    }
  }
}
template <typename T>
__device__ __forceinline__ ss::u32x4 pack(const float (&f)[16 / sizeof(T)]) {
  ss::u32x4 w;
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = __builtin_bit_cast(uint32_t, f[e]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = ss::Elem<T>::pack2(f[2 * e], f[2 * e + 1]);
  }
  return w;
}

struct NormArgs {
  const char* x;
  const char* res;
  const char* w;
  char* y;
  int64_t x_stride, r_stride, y_stride;  // bytes
  int cols;
  float eps;
};

// PPT 16-byte pieces per thread, register-resident (cols <= 256 * PPT * EPP)
template <typename T, int PPT>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const NormArgs a) {
  constexpr int EPP = 16 / sizeof(T);
  __shared__ float s_part[4];
  const int64_t row = blockIdx.x;
  const char* xr = a.x + row * a.x_stride;
  const char* rr = a.res ? a.res + row * a.r_stride : nullptr;
  const int pieces = a.cols / EPP;
  float v[PPT][EPP];
  float ss = 0.f;
#pragma unroll
  for (int u = 0; u < PPT; ++u) {
    const int pc = threadIdx.x + 256 * u;
    if (pc < pieces) {
      unpack<T>(*reinterpret_cast<const ss::u32x4*>(xr + (int64_t)pc * 16), v[u]);
      if (rr) {
        float rv[EPP];
        unpack<T>(*reinterpret_cast<const ss::u32x4*>(rr + (int64_t)pc * 16), rv);
#pragma unroll
        for (int e = 0; e < EPP; ++e) v[u][e] = Rnd<T>::r(pin(v[u][e] + rv[e]));
      }
#pragma unroll
      for (int e = 0; e < EPP; ++e) ss += pin(v[u][e] * v[u][e]);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float mean = (s_part[0] + s_part[1] + s_part[2] + s_part[3]) / (float)a.cols;
  const float rstd = 1.0f / __builtin_sqrtf(mean + a.eps);
#pragma unroll
  for (int u = 0; u < PPT; ++u) {
    const int pc = threadIdx.x + 256 * u;
    if (pc < pieces) {
      float wv[EPP], o[EPP];
      unpack<T>(*reinterpret_cast<const ss::u32x4*>(a.w + (int64_t)pc * 16), wv);
#pragma unroll
      for (int e = 0; e < EPP; ++e) o[e] = Rnd<T>::r(pin(wv[e] * Rnd<T>::r(pin(v[u][e] * rstd))));
      *reinterpret_cast<ss::u32x4*>(a.y + row * a.y_stride + (int64_t)pc * 16) = pack<T>(o);
    }
  }
}

// Rows longer than the register-resident variants hold (more than 256 * 8 pieces):
// two passes over the row in memory -- the sum of squares, then the normalised
// output -- reading x (and the residual) twice. Each thread adds its pieces in the
// same order as rmsnorm_kernel (pc = tid, tid + 256, ...), then the same reduction.
template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_long_kernel(const NormArgs a) {
  constexpr int EPP = 16 / sizeof(T);
  __shared__ float s_part[4];
  const int64_t row = blockIdx.x;
  const char* xr = a.x + row * a.x_stride;
  const char* rr = a.res ? a.res + row * a.r_stride : nullptr;
  const int pieces = a.cols / EPP;
  auto load_row = [&](int pc, float (&v)[EPP]) {
    unpack<T>(*reinterpret_cast<const ss::u32x4*>(xr + (int64_t)pc * 16), v);
    if (rr) {
      float rv[EPP];
      unpack<T>(*reinterpret_cast<const ss::u32x4*>(rr + (int64_t)pc * 16), rv);
#pragma unroll
      for (int e = 0; e < EPP; ++e) v[e] = Rnd<T>::r(pin(v[e] + rv[e]));
    }
  };
  float ss = 0.f;
  for (int pc = threadIdx.x; pc < pieces; pc += 256) {
    float v[EPP];
    load_row(pc, v);
#pragma unroll
    for (int e = 0; e < EPP; ++e) ss += pin(v[e] * v[e]);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float mean = (s_part[0] + s_part[1] + s_part[2] + s_part[3]) / (float)a.cols;
  const float rstd = 1.0f / __builtin_sqrtf(mean + a.eps);
  for (int pc = threadIdx.x; pc < pieces; pc += 256) {
    float v[EPP], wv[EPP], o[EPP];
    load_row(pc, v);
    unpack<T>(*reinterpret_cast<const ss::u32x4*>(a.w + (int64_t)pc * 16), wv);
#pragma unroll
    for (int e = 0; e < EPP; ++e) o[e] = Rnd<T>::r(pin(wv[e] * Rnd<T>::r(pin(v[e] * rstd))));
    *reinterpret_cast<ss::u32x4*>(a.y + row * a.y_stride + (int64_t)pc * 16) = pack<T>(o);
  }
}

struct SwigluArgs {
  const char* g;
  const char* u;
  char* o;
  int64_t rows;
  int pieces;  // per row
  int64_t g_stride, u_stride, o_stride;  // bytes
};

template <typename T>
__global__ __launch_bounds__(256) void swiglu_kernel(const SwigluArgs a) {
  constexpr int EPP = 16 / sizeof(T);
  const int64_t total = a.rows * a.pieces;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / a.pieces;
    const int64_t pc = i - r * a.pieces;
    float g[EPP], u[EPP], o[EPP];
    unpack<T>(*reinterpret_cast<const ss::u32x4*>(a.g + r * a.g_stride + pc * 16), g);
    unpack<T>(*reinterpret_cast<const ss::u32x4*>(a.u + r * a.u_stride + pc * 16), u);
#pragma unroll
    for (int e = 0; e < EPP; ++e) {
      const float s = Rnd<T>::r(pin(g[e] / pin(1.0f + expf(-g[e]))));
      o[e] = Rnd<T>::r(pin(s * u[e]));
    }
    *reinterpret_cast<ss::u32x4*>(a.o + r * a.o_stride + pc * 16) = pack<T>(o);
  }
}

bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

template <typename T>
int launch_rmsnorm(const NormArgs& a, int64_t rows, hipStream_t s) {
  constexpr int EPP = 16 / sizeof(T);
  const int pieces = a.cols / EPP;
  if (pieces <= 256)
    hipLaunchKernelGGL((rmsnorm_kernel<T, 1>), dim3((unsigned)rows), dim3(256), 0, s, a);
  else if (pieces <= 512)
    hipLaunchKernelGGL((rmsnorm_kernel<T, 2>), dim3((unsigned)rows), dim3(256), 0, s, a);
  else if (pieces <= 1024)
    hipLaunchKernelGGL((rmsnorm_kernel<T, 4>), dim3((unsigned)rows), dim3(256), 0, s, a);
  else if (pieces <= 2048)
    hipLaunchKernelGGL((rmsnorm_kernel<T, 8>), dim3((unsigned)rows), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((rmsnorm_long_kernel<T>), dim3((unsigned)rows), dim3(256), 0, s, a);
  return ss_host::launch_status("rmsnorm");
}

}  // namespace

extern "C" int ss_rmsnorm(const void* x, const void* residual, const void* weight, void* out, int64_t rows,
                          int cols, int64_t x_stride, int64_t r_stride, int64_t o_stride, float eps, int dtype,
                          void* stream) {
  const char* who = "rmsnorm";
  if (rows < 0 || cols < 0) {
    ss_host::set_error("%s: negative extent", who);
    return SS_ERR_INVALID;
  }
  if (rows == 0 || cols == 0) return SS_OK;
  if (!x || !weight || !out) {
    ss_host::set_error("%s: null pointer", who);
    return SS_ERR_INVALID;
  }
  if (dtype != SS_DTYPE_BF16 && dtype != SS_DTYPE_F16 && dtype != SS_DTYPE_F32) {
    ss_host::set_error("%s: dtype code %d not supported", who, dtype);
    return SS_ERR_UNSUPPORTED;
  }
  const int es = dtype == SS_DTYPE_F32 ? 4 : 2;
  const int epp = 16 / es;
  if (cols % epp != 0 || !al16(x) || !al16(weight) || !al16(out) || (residual && !al16(residual)) ||
      (x_stride * es) % 16 || (o_stride * es) % 16 || (residual && (r_stride * es) % 16) || rows > 0x7fffffff) {
    ss_host::set_error("%s: rows must be 16-byte aligned with %d-element multiples", who, epp);
    return SS_ERR_UNSUPPORTED;
  }
  NormArgs a;
  a.x = (const char*)x;
  a.res = (const char*)residual;
  a.w = (const char*)weight;
  a.y = (char*)out;
  a.x_stride = x_stride * es;
  a.r_stride = r_stride * es;
  a.y_stride = o_stride * es;
  a.cols = cols;
  a.eps = eps;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == SS_DTYPE_BF16) return launch_rmsnorm<ss::bf16_t>(a, rows, s);
  if (dtype == SS_DTYPE_F16) return launch_rmsnorm<ss::f16_t>(a, rows, s);
  return launch_rmsnorm<float>(a, rows, s);
}

extern "C" int ss_swiglu(const void* gate, const void* up, void* out, int64_t rows, int cols, int64_t g_stride,
                         int64_t u_stride, int64_t o_stride, int dtype, void* stream) {
  const char* who = "swiglu";
  if (rows < 0 || cols < 0) {
    ss_host::set_error("%s: negative extent", who);
    return SS_ERR_INVALID;
  }
  if (rows == 0 || cols == 0) return SS_OK;
  if (!gate || !up || !out) {
    ss_host::set_error("%s: null pointer", who);
    return SS_ERR_INVALID;
  }
  if (dtype != SS_DTYPE_BF16 && dtype != SS_DTYPE_F16 && dtype != SS_DTYPE_F32) {
    ss_host::set_error("%s: dtype code %d not supported", who, dtype);
    return SS_ERR_UNSUPPORTED;
  }
  const int es = dtype == SS_DTYPE_F32 ? 4 : 2;
  const int epp = 16 / es;
  if (cols % epp != 0 || !al16(gate) || !al16(up) || !al16(out) || (g_stride * es) % 16 || (u_stride * es) % 16 ||
      (o_stride * es) % 16) {
    ss_host::set_error("%s: rows must be 16-byte aligned with %d-element multiples", who, epp);
    return SS_ERR_UNSUPPORTED;
  }
  SwigluArgs a;
  a.g = (const char*)gate;
  a.u = (const char*)up;
  a.o = (char*)out;
  a.rows = rows;
  a.pieces = cols / epp;
  a.g_stride = g_stride * es;
  a.u_stride = u_stride * es;
  a.o_stride = o_stride * es;
  int64_t blocks = (rows * a.pieces + 255) / 256;
  const int64_t cap = (int64_t)ss_host::device_cu_count() * 16;
  if (blocks > cap) blocks = cap;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == SS_DTYPE_BF16)
    hipLaunchKernelGGL(swiglu_kernel<ss::bf16_t>, dim3((unsigned)blocks), dim3(256), 0, s, a);
  else if (dtype == SS_DTYPE_F16)
    hipLaunchKernelGGL(swiglu_kernel<ss::f16_t>, dim3((unsigned)blocks), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(swiglu_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, s, a);
  return ss_host::launch_status(who);
}
