// KV-cache slot-mapping scatter (reshape_and_cache) for gfx950.
//
// Semantics: slipstream/kernels/attention_ref.py:21-39 (index_put of token n's
// [n_kv, D] row into kv_cache[layer, 0/1, slot // bs, slot % bs]) with the skip
// of negative slots from slipstream/kernels/triton_paged.py:70-71. The copy is a
// byte copy, so it is bit exact for every element type.
//
// Work layout: one thread moves one CHUNK-byte piece of one (token, head) row of
// both K and V. Consecutive threads take consecutive pieces of a row, then the
// next head, then the next token, so a wavefront reads and writes whole rows
// (256 B per row for D=128 bf16) with 16-byte accesses on both sides.
#include "ss_common.h"

namespace {

template <int CHUNK>
struct Piece;
template <>
struct Piece<16> {
  typedef ss::u32x4 type;
};
template <>
struct Piece<8> {
  typedef ss::u32x2 type;
};
template <>
struct Piece<4> {
  typedef uint32_t type;
};
template <>
struct Piece<2> {
  typedef uint16_t type;
};

struct ScatterArgs {
  const char* k;
  const char* v;
  char* kc;
  char* vc;
  const int64_t* slots;
  int64_t n_tok;
  int64_t n_inner;
  int64_t k_so, k_si, k_sh;  // byte strides
  int64_t v_so, v_si, v_sh;
  int64_t c_sb, c_so, c_sh;
  int64_t num_slots;
  int n_kv;
  int pieces_per_row;
  int bs_shift;  // block_size = 1 << bs_shift when >= 0
  int block_size;
};

template <int CHUNK>
__global__ __launch_bounds__(256) void scatter_kernel(const ScatterArgs a) {
  typedef typename Piece<CHUNK>::type P;
  const int64_t total = a.n_tok * a.n_kv * a.pieces_per_row;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int piece = (int)(i % a.pieces_per_row);
    const int64_t row = i / a.pieces_per_row;
    const int h = (int)(row % a.n_kv);
    const int64_t tok = row / a.n_kv;
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
    const int64_t to = tok / a.n_inner, ti = tok - to * a.n_inner;
    const int64_t pb = (int64_t)piece * CHUNK;
    const P kv = *reinterpret_cast<const P*>(a.k + to * a.k_so + ti * a.k_si + h * a.k_sh + pb);
    const P vv = *reinterpret_cast<const P*>(a.v + to * a.v_so + ti * a.v_si + h * a.v_sh + pb);
    const int64_t dst = blk * a.c_sb + off * a.c_so + h * a.c_sh + pb;
    *reinterpret_cast<P*>(a.kc + dst) = kv;
    *reinterpret_cast<P*>(a.vc + dst) = vv;
  }
}

template <int CHUNK>
int launch_scatter(const ScatterArgs& a, hipStream_t stream) {
  const int64_t total = a.n_tok * a.n_kv * a.pieces_per_row;
  const int threads = 256;
  int64_t blocks = (total + threads - 1) / threads;
  const int64_t cap = (int64_t)ss_host::device_cu_count() * 32;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(scatter_kernel<CHUNK>, dim3((unsigned)blocks), dim3(threads), 0, stream, a);
  return ss_host::launch_status("reshape_and_cache");
}

bool aligned(const void* p, int64_t bytes) { return ((uintptr_t)p % (uintptr_t)bytes) == 0; }

}  // namespace

extern "C" int ss_reshape_and_cache(const void* k, const void* v, void* k_cache, void* v_cache,
                                    const int64_t* slot_mapping, int64_t n_outer, int64_t n_inner,
                                    int n_kv, int head_dim, int block_size, int64_t num_slots,
                                    const int64_t k_strides[3], const int64_t v_strides[3],
                                    const int64_t c_strides[3], int elem_bytes, void* stream) {
  if (n_outer < 0 || n_inner < 0 || n_kv < 0 || head_dim < 0) {
    ss_host::set_error("reshape_and_cache: negative extent");
    return SS_ERR_INVALID;
  }
  if (block_size < 1) {
    ss_host::set_error("reshape_and_cache: block_size must be >= 1, got %d", block_size);
    return SS_ERR_INVALID;
  }
  if (elem_bytes != 2 && elem_bytes != 4) {
    ss_host::set_error("reshape_and_cache: element size %d not supported", elem_bytes);
    return SS_ERR_UNSUPPORTED;
  }
  const int64_t n_tok = n_outer * n_inner;
  if (n_tok == 0 || n_kv == 0 || head_dim == 0) return SS_OK;
  if (!k || !v || !k_cache || !v_cache || !slot_mapping) {
    ss_host::set_error("reshape_and_cache: null pointer");
    return SS_ERR_INVALID;
  }
  ScatterArgs a;
  a.k = (const char*)k;
  a.v = (const char*)v;
  a.kc = (char*)k_cache;
  a.vc = (char*)v_cache;
  a.slots = slot_mapping;
  a.n_tok = n_tok;
  a.n_inner = n_inner > 0 ? n_inner : 1;
  a.k_so = k_strides[0] * elem_bytes;
  a.k_si = k_strides[1] * elem_bytes;
  a.k_sh = k_strides[2] * elem_bytes;
  a.v_so = v_strides[0] * elem_bytes;
  a.v_si = v_strides[1] * elem_bytes;
  a.v_sh = v_strides[2] * elem_bytes;
  a.c_sb = c_strides[0] * elem_bytes;
  a.c_so = c_strides[1] * elem_bytes;
  a.c_sh = c_strides[2] * elem_bytes;
  a.num_slots = num_slots;
  a.n_kv = n_kv;
  a.block_size = block_size;
  a.bs_shift = ((block_size & (block_size - 1)) == 0) ? __builtin_ctz((unsigned)block_size) : -1;

  const int64_t row_bytes = (int64_t)head_dim * elem_bytes;
  // Widest piece that divides the row and every base/stride alignment.
  int chunk = 16;
  while (chunk > elem_bytes) {
    bool ok = (row_bytes % chunk) == 0 && aligned(k, chunk) && aligned(v, chunk) &&
              aligned(k_cache, chunk) && aligned(v_cache, chunk);
    const int64_t st[9] = {a.k_so, a.k_si, a.k_sh, a.v_so, a.v_si, a.v_sh, a.c_sb, a.c_so, a.c_sh};
    for (int i = 0; i < 9 && ok; ++i) ok = (st[i] % chunk) == 0;
    if (ok) break;
    chunk >>= 1;
  }
  a.pieces_per_row = (int)(row_bytes / chunk);
  hipStream_t s = (hipStream_t)stream;
  switch (chunk) {
    case 16:
      return launch_scatter<16>(a, s);
    case 8:
      return launch_scatter<8>(a, s);
    case 4:
      return launch_scatter<4>(a, s);
    default:
      return launch_scatter<2>(a, s);
  }
}
