// Fused rotary embedding + KV scatter for gfx950.
//
// Semantics: slipstream/models/layers/rope.py:13-36 (apply_rotary_pos_emb:
// x_embed = x * cos + rotate_half(x) * sin, rotate_half(x) = cat(-x2, x1)) on Q and
// K, followed by the KV scatter of slipstream/kernels/attention_ref.py:21-39 (with
// the skip of negative slots, triton_paged.py:70-71) as the attention layer runs
// them (slipstream/models/layers/attention.py:163,171-174). The rotated K goes
// straight into the cache: the reference writes k_embed to memory and reads it
// back for the scatter; here K is read once and written once.
//
// Arithmetic follows the reference's dtype sequence exactly: each torch
// elementwise op computes in fp32 and rounds to the tensor dtype, so
//   out[i]       = r( r(x[i] * cos[i])             + r(-x[i + D/2] * sin[i]) )
//   out[i + D/2] = r( r(x[i + D/2] * cos[i + D/2]) + r(x[i] * sin[i + D/2]) )
// with r() the round to bf16/fp16 (nearest even); for fp32 tensors the products
// and the sum are separately rounded fp32 operations (no fused multiply-add).
// The result is bit identical to the reference for every input.
//
// Work layout: one thread takes EPP consecutive elements of the first half of a
// row and the matching EPP of the second half (16-byte pieces when the strides
// allow), of a Q row (written to q_out), a K row (written rotated into the cache)
// or a V row (copied into the cache). Rows of one token are consecutive, so a
// wavefront reads and writes whole head rows.
#include "ss_common.h"

namespace {

struct RopeArgs {
  const char* q;
  const char* k;
  const char* v;
  const char* cs;  // cos
  const char* sn;  // sin
  char* qo;
  char* kc;
  char* vc;
  const int64_t* slots;
  int64_t n_tok, n_inner;  // token n = o * n_inner + i
  // byte strides (outer, inner, head)
  int64_t q_so, q_si, q_sh, k_so, k_si, k_sh, v_so, v_si, v_sh, o_so, o_si, o_sh;
  int64_t c_so, c_si, s_so, s_si;  // cos / sin token strides
  int64_t c_sb, c_sp, c_sh;        // cache strides (block, position, head)
  int64_t num_slots;
  int n_q, n_kv;
  int half_bytes;     // bytes of half a row
  int pieces;         // pieces per half row
  int bs_shift, block_size;
};

// An fp32 result the compiler may not narrow to 16-bit arithmetic or fuse with the
// next operation: without the pin, fp-contract turns a product and the following sum
// into one f16 FMA, which skips the product's rounding the reference performs.
__device__ __forceinline__ float pin32(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

template <typename T>
struct Num;
template <>
struct Num<ss::bf16_t> {
  static __device__ __forceinline__ float get(uint32_t w, int hi) { return __builtin_bit_cast(float, hi ? (w & 0xFFFF0000u) : (w << 16)); }
  static __device__ __forceinline__ float mul(float a, float b) { return (float)(ss::bf16_t)pin32(__fmul_rn(a, b)); }
  static __device__ __forceinline__ float add(float a, float b) { return (float)(ss::bf16_t)pin32(__fadd_rn(a, b)); }
};
template <>
struct Num<ss::f16_t> {
  static __device__ __forceinline__ float get(uint32_t w, int hi) {
    return (float)__builtin_bit_cast(ss::f16_t, (uint16_t)(hi ? (w >> 16) : (w & 0xFFFFu)));
  }
  static __device__ __forceinline__ float mul(float a, float b) { return (float)(ss::f16_t)pin32(__fmul_rn(a, b)); }
  static __device__ __forceinline__ float add(float a, float b) { return (float)(ss::f16_t)pin32(__fadd_rn(a, b)); }
};
template <>
struct Num<float> {
  static __device__ __forceinline__ float mul(float a, float b) { return pin32(__fmul_rn(a, b)); }
  static __device__ __forceinline__ float add(float a, float b) { return pin32(__fadd_rn(a, b)); }
};

// EPP elements of type T at p <-> floats
template <typename T, int EPP>
__device__ __forceinline__ void load_elems(const char* p, float (&f)[EPP]) {
  if constexpr (sizeof(T) == 4) {
    if constexpr (EPP == 4) {
      const ss::u32x4 w = *reinterpret_cast<const ss::u32x4*>(p);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // through a scalar: bit_cast of a vector element in place reads element 0
        const uint32_t u = w[e];
        f[e] = __builtin_bit_cast(float, u);
      }
    } else {
      f[0] = *reinterpret_cast<const float*>(p);
    }
  } else {
    if constexpr (EPP == 8) {
      const ss::u32x4 w = *reinterpret_cast<const ss::u32x4*>(p);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = Num<T>::get(w[e >> 1], e & 1);
    } else {
      f[0] = Num<T>::get(*reinterpret_cast<const uint16_t*>(p), 0);
    }
  }
}
template <typename T, int EPP>
__device__ __forceinline__ void store_elems(char* p, const float (&f)[EPP]) {
  if constexpr (sizeof(T) == 4) {
    if constexpr (EPP == 4) {
      *reinterpret_cast<ss::u32x4*>(p) = ss::u32x4{__builtin_bit_cast(uint32_t, f[0]), __builtin_bit_cast(uint32_t, f[1]),
                                                   __builtin_bit_cast(uint32_t, f[2]), __builtin_bit_cast(uint32_t, f[3])};
    } else {
      *reinterpret_cast<float*>(p) = f[0];
    }
  } else {
    if constexpr (EPP == 8) {
      ss::u32x4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = ss::Elem<T>::pack2(f[2 * e], f[2 * e + 1]);
      *reinterpret_cast<ss::u32x4*>(p) = w;
    } else {
      *reinterpret_cast<T*>(p) = (T)f[0];
    }
  }
}

// copy of EPP elements (V rows): raw bytes
template <typename T, int EPP>
__device__ __forceinline__ void copy_elems(char* d, const char* s) {
  if constexpr (EPP * sizeof(T) == 16)
    *reinterpret_cast<ss::u32x4*>(d) = *reinterpret_cast<const ss::u32x4*>(s);
  else
    *reinterpret_cast<T*>(d) = *reinterpret_cast<const T*>(s);
}

template <typename T, int EPP>
__global__ __launch_bounds__(256) void rope_cache_kernel(const RopeArgs a) {
  const int rows = a.n_q + 2 * a.n_kv;
  const int64_t total = a.n_tok * rows * a.pieces;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int piece = (int)(i % a.pieces);
    const int64_t rt = i / a.pieces;
    const int h = (int)(rt % rows);
    const int64_t tok = rt / rows;
    const int64_t to = tok / a.n_inner, ti = tok - to * a.n_inner;
    const int64_t pb = (int64_t)piece * EPP * (int64_t)sizeof(T);
    char* dst;
    const char* src;
    bool rotate = true;
    if (h < a.n_q) {
      src = a.q + to * a.q_so + ti * a.q_si + (int64_t)h * a.q_sh;
      dst = a.qo + to * a.o_so + ti * a.o_si + (int64_t)h * a.o_sh;
    } else {
      const int64_t slot = a.slots[tok];
      if (slot < 0 || slot >= a.num_slots) continue;
      int64_t blk, off;
      if (a.bs_shift >= 0) {
        blk = slot >> a.bs_shift;
        off = slot & ((int64_t)a.block_size - 1);
      } else {
        blk = slot / a.block_size;
        off = slot - blk * a.block_size;
      }
      const bool is_k = h < a.n_q + a.n_kv;
      const int hk = is_k ? h - a.n_q : h - a.n_q - a.n_kv;
      const int64_t cpos = blk * a.c_sb + off * a.c_sp + (int64_t)hk * a.c_sh;
      if (is_k) {
        src = a.k + to * a.k_so + ti * a.k_si + (int64_t)hk * a.k_sh;
        dst = a.kc + cpos;
      } else {
        src = a.v + to * a.v_so + ti * a.v_si + (int64_t)hk * a.v_sh;
        dst = a.vc + cpos;
        rotate = false;
      }
    }
    if (!rotate) {
      copy_elems<T, EPP>(dst + pb, src + pb);
      copy_elems<T, EPP>(dst + a.half_bytes + pb, src + a.half_bytes + pb);
      continue;
    }
    const char* cr = a.cs + to * a.c_so + ti * a.c_si;
    const char* sr = a.sn + to * a.s_so + ti * a.s_si;
    float x1[EPP], x2[EPP], c1[EPP], c2[EPP], s1[EPP], s2[EPP], o1[EPP], o2[EPP];
    load_elems<T, EPP>(src + pb, x1);
    load_elems<T, EPP>(src + a.half_bytes + pb, x2);
    load_elems<T, EPP>(cr + pb, c1);
    load_elems<T, EPP>(cr + a.half_bytes + pb, c2);
    load_elems<T, EPP>(sr + pb, s1);
    load_elems<T, EPP>(sr + a.half_bytes + pb, s2);
#pragma unroll
    for (int e = 0; e < EPP; ++e) {
      o1[e] = Num<T>::add(Num<T>::mul(x1[e], c1[e]), Num<T>::mul(-x2[e], s1[e]));
      o2[e] = Num<T>::add(Num<T>::mul(x2[e], c2[e]), Num<T>::mul(x1[e], s2[e]));
    }
    store_elems<T, EPP>(dst + pb, o1);
    store_elems<T, EPP>(dst + a.half_bytes + pb, o2);
  }
}

template <typename T, int EPP>
int launch_rope(const RopeArgs& a, hipStream_t stream) {
  const int64_t total = a.n_tok * (a.n_q + 2 * a.n_kv) * a.pieces;
  int64_t blocks = (total + 255) / 256;
  const int64_t cap = (int64_t)ss_host::device_cu_count() * 32;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL((rope_cache_kernel<T, EPP>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
  return ss_host::launch_status("rope_and_cache");
}

bool al(const void* p, int64_t b) { return ((uintptr_t)p % (uintptr_t)b) == 0; }

}  // namespace

extern "C" int ss_rope_and_cache(const void* q, const void* k, const void* v, const void* cos, const void* sin,
                                 void* q_out, void* k_cache, void* v_cache, const int64_t* slot_mapping,
                                 int64_t n_outer, int64_t n_inner, int n_q, int n_kv, int head_dim, int block_size,
                                 int64_t num_slots, const int64_t q_strides[3], const int64_t k_strides[3],
                                 const int64_t v_strides[3], const int64_t o_strides[3], const int64_t cos_strides[2],
                                 const int64_t sin_strides[2], const int64_t c_strides[3], int dtype, void* stream) {
  const char* who = "rope_and_cache";
  if (n_outer < 0 || n_inner < 0 || n_q < 0 || n_kv < 0 || head_dim < 0) {
    ss_host::set_error("%s: negative extent", who);
    return SS_ERR_INVALID;
  }
  if (head_dim % 2 != 0) {
    ss_host::set_error("%s: head_dim must be even, got %d", who, head_dim);
    return SS_ERR_INVALID;
  }
  if (block_size < 1) {
    ss_host::set_error("%s: block_size must be >= 1, got %d", who, block_size);
    return SS_ERR_INVALID;
  }
  if (dtype != SS_DTYPE_BF16 && dtype != SS_DTYPE_F16 && dtype != SS_DTYPE_F32) {
    ss_host::set_error("%s: dtype code %d not supported", who, dtype);
    return SS_ERR_UNSUPPORTED;
  }
  const int64_t n_tok = n_outer * n_inner;
  if (n_tok == 0 || head_dim == 0 || (n_q == 0 && n_kv == 0)) return SS_OK;
  if (!q_strides || !k_strides || !v_strides || !o_strides || !cos_strides || !sin_strides || !c_strides ||
      !cos || !sin || (n_q > 0 && (!q || !q_out)) || (n_kv > 0 && (!k || !v || !k_cache || !v_cache || !slot_mapping))) {
    ss_host::set_error("%s: null pointer", who);
    return SS_ERR_INVALID;
  }
  const int es = dtype == SS_DTYPE_F32 ? 4 : 2;
  RopeArgs a;
  a.q = (const char*)q;
  a.k = (const char*)k;
  a.v = (const char*)v;
  a.cs = (const char*)cos;
  a.sn = (const char*)sin;
  a.qo = (char*)q_out;
  a.kc = (char*)k_cache;
  a.vc = (char*)v_cache;
  a.slots = slot_mapping;
  a.n_tok = n_tok;
  a.n_inner = n_inner > 0 ? n_inner : 1;
  a.q_so = q_strides[0] * es, a.q_si = q_strides[1] * es, a.q_sh = q_strides[2] * es;
  a.k_so = k_strides[0] * es, a.k_si = k_strides[1] * es, a.k_sh = k_strides[2] * es;
  a.v_so = v_strides[0] * es, a.v_si = v_strides[1] * es, a.v_sh = v_strides[2] * es;
  a.o_so = o_strides[0] * es, a.o_si = o_strides[1] * es, a.o_sh = o_strides[2] * es;
  a.c_so = cos_strides[0] * es, a.c_si = cos_strides[1] * es;
  a.s_so = sin_strides[0] * es, a.s_si = sin_strides[1] * es;
  a.c_sb = c_strides[0] * es, a.c_sp = c_strides[1] * es, a.c_sh = c_strides[2] * es;
  a.num_slots = num_slots;
  a.n_q = n_q;
  a.n_kv = n_kv;
  a.half_bytes = head_dim / 2 * es;
  a.block_size = block_size;
  a.bs_shift = ((block_size & (block_size - 1)) == 0) ? __builtin_ctz((unsigned)block_size) : -1;
  // 16-byte pieces when half a row and every base and stride allow them
  bool wide = a.half_bytes % 16 == 0;
  const void* ptrs[10] = {q, k, v, cos, sin, q_out, k_cache, v_cache, nullptr, nullptr};
  for (int i = 0; i < 8 && wide; ++i) wide = !ptrs[i] || al(ptrs[i], 16);
  const int64_t st[19] = {a.q_so, a.q_si, a.q_sh, a.k_so, a.k_si, a.k_sh, a.v_so, a.v_si, a.v_sh, a.o_so,
                          a.o_si, a.o_sh, a.c_so, a.c_si, a.s_so, a.s_si, a.c_sb, a.c_sp, a.c_sh};
  for (int i = 0; i < 19 && wide; ++i) wide = st[i] % 16 == 0;
  const int epp = wide ? 16 / es : 1;
  a.pieces = head_dim / 2 / epp;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == SS_DTYPE_BF16) return wide ? launch_rope<ss::bf16_t, 8>(a, s) : launch_rope<ss::bf16_t, 1>(a, s);
  if (dtype == SS_DTYPE_F16) return wide ? launch_rope<ss::f16_t, 8>(a, s) : launch_rope<ss::f16_t, 1>(a, s);
  return wide ? launch_rope<float, 4>(a, s) : launch_rope<float, 1>(a, s);
}
