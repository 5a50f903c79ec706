// KV page copies for gfx950: copy-on-write inside one cache, and swap between the
// device cache and a pinned host cache.
//
// Semantics: slipstream/kernels/attention_ref.py:92-94 (copy_blocks_ref: for each
// (src, dst), kv_cache[:, :, dst] <- kv_cache[:, :, src] over every layer and K/V,
// the copy slipstream/memory/block_manager.py:297-298 makes on copy-on-write) and
// the swap copies of block_manager.py:196-200 (out: cpu[:, :, cpu_id] <-
// gpu[:, :, gpu_id]) and :220-225 (in: the reverse). A page is one (layer, K/V,
// block) slice [block_size, n_kv, D]: page_bytes contiguous bytes. The copy is a
// byte copy, bit exact for every element type.
//
// Work layout: blockIdx.y = plane (layer, K/V); blockIdx.x = (pair, piece of the
// page). A thread moves kUnroll pieces of VEC bytes (16 unless a stride or the
// page size forbids it), all loads before all stores, so a workgroup moves
// 256 * kUnroll * VEC contiguous bytes of one page with every load in flight at
// once. A pinned host page is read or written through its device mapping (the
// copy then runs at the host link's rate). Pairs with a block id outside its
// cache are skipped: the caller validates ids on the host, and this only keeps a
// bad id from writing out of bounds.
#include "ss_common.h"

namespace {

constexpr int kUnroll = 4;

struct CopyArgs {
  char* dst;
  const char* src;
  int64_t dst_plane, dst_block;  // byte strides
  int64_t src_plane, src_block;
  int64_t dst_blocks, src_blocks;
  int64_t page_bytes;
  const int64_t* pairs;  // [n_pairs, 2]: (source block, destination block)
  int64_t wg_per_page;
};

template <int VEC>
struct Vec;
template <>
struct Vec<16> {
  typedef ss::u32x4 type;
};
template <>
struct Vec<4> {
  typedef uint32_t type;
};
template <>
struct Vec<1> {
  typedef uint8_t type;
};

template <int VEC>
__global__ __launch_bounds__(256) void copy_pages_kernel(const CopyArgs a) {
  typedef typename Vec<VEC>::type P;
  const int64_t job = blockIdx.x;
  const int64_t pair = job / a.wg_per_page;
  const int64_t part = job - pair * a.wg_per_page;
  const int64_t s = a.pairs[2 * pair], d = a.pairs[2 * pair + 1];
  if (s < 0 || s >= a.src_blocks || d < 0 || d >= a.dst_blocks) return;
  const char* sp = a.src + (int64_t)blockIdx.y * a.src_plane + s * a.src_block;
  char* dp = a.dst + (int64_t)blockIdx.y * a.dst_plane + d * a.dst_block;
  const int64_t base = part * (256 * kUnroll * VEC) + (int64_t)threadIdx.x * VEC;
  P v[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t off = base + (int64_t)u * 256 * VEC;
    if (off < a.page_bytes) v[u] = *reinterpret_cast<const P*>(sp + off);
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t off = base + (int64_t)u * 256 * VEC;
    if (off < a.page_bytes) *reinterpret_cast<P*>(dp + off) = v[u];
  }
}

bool aligned_to(int64_t v, int a) { return v % a == 0; }

// Device address of p: itself for device memory, the device mapping for pinned host
// memory; nullptr (with the error set) for memory the device cannot reach.
void* device_address(void* p, const char* what) {
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
    (void)hipGetLastError();  // the failed query must not be reported by a later call
    ss_host::set_error("copy_blocks: %s is not device memory or pinned host memory", what);
    return nullptr;
  }
  if (attr.type == hipMemoryTypeUnregistered) {
    ss_host::set_error("copy_blocks: %s is pageable host memory (pin it: hipHostMalloc, pin_memory=True)", what);
    return nullptr;
  }
  if (attr.type == hipMemoryTypeHost) {
    if (!attr.devicePointer) {
      ss_host::set_error("copy_blocks: %s is host memory without a device mapping", what);
      return nullptr;
    }
    // hostPointer and devicePointer name the same byte (the allocation's start or p
    // itself, by runtime version): keep p's offset from it
    if (!attr.hostPointer) return attr.devicePointer;
    return (char*)attr.devicePointer + ((char*)p - (char*)attr.hostPointer);
  }
  return p;
}

}  // namespace

extern "C" int ss_copy_blocks(void* dst, const void* src, int64_t planes, int64_t dst_plane_stride,
                              int64_t dst_block_stride, int64_t dst_blocks, int64_t src_plane_stride,
                              int64_t src_block_stride, int64_t src_blocks, int64_t page_bytes,
                              const int64_t* pairs, int64_t n_pairs, void* stream) {
  const char* who = "copy_blocks";
  if (planes < 0 || n_pairs < 0 || page_bytes < 0 || dst_blocks < 0 || src_blocks < 0) {
    ss_host::set_error("%s: negative extent", who);
    return SS_ERR_INVALID;
  }
  if (planes == 0 || n_pairs == 0 || page_bytes == 0) return SS_OK;
  if (!dst || !src || !pairs) {
    ss_host::set_error("%s: null pointer", who);
    return SS_ERR_INVALID;
  }
  if (planes > 65535) {
    ss_host::set_error("%s: %lld planes exceed the grid", who, (long long)planes);
    return SS_ERR_UNSUPPORTED;
  }
  CopyArgs a;
  a.dst = (char*)device_address(dst, "destination");
  if (!a.dst) return SS_ERR_INVALID;
  a.src = (const char*)device_address(const_cast<void*>(src), "source");
  if (!a.src) return SS_ERR_INVALID;
  a.dst_plane = dst_plane_stride;
  a.dst_block = dst_block_stride;
  a.src_plane = src_plane_stride;
  a.src_block = src_block_stride;
  a.dst_blocks = dst_blocks;
  a.src_blocks = src_blocks;
  a.page_bytes = page_bytes;
  a.pairs = (const int64_t*)device_address(const_cast<int64_t*>(pairs), "pairs");
  if (!a.pairs) return SS_ERR_INVALID;
  int vec = 16;
  while (vec > 1) {
    const int64_t v[7] = {(int64_t)(uintptr_t)a.dst, (int64_t)(uintptr_t)a.src, dst_plane_stride,
                          dst_block_stride, src_plane_stride, src_block_stride, page_bytes};
    bool ok = true;
    for (int i = 0; i < 7 && ok; ++i) ok = aligned_to(v[i], vec);
    if (ok) break;
    vec = vec == 16 ? 4 : 1;
  }
  a.wg_per_page = (page_bytes + 256LL * kUnroll * vec - 1) / (256LL * kUnroll * vec);
  const int64_t jobs = n_pairs * a.wg_per_page;
  if (jobs > 0x7fffffff) {
    ss_host::set_error("%s: %lld page pieces exceed the grid", who, (long long)jobs);
    return SS_ERR_UNSUPPORTED;
  }
  const dim3 grid((unsigned)jobs, (unsigned)planes);
  hipStream_t s = (hipStream_t)stream;
  if (vec == 16)
    hipLaunchKernelGGL(copy_pages_kernel<16>, grid, dim3(256), 0, s, a);
  else if (vec == 4)
    hipLaunchKernelGGL(copy_pages_kernel<4>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(copy_pages_kernel<1>, grid, dim3(256), 0, s, a);
  return ss_host::launch_status(who);
}
