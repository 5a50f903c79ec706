// Packed-step metadata built on the device for gfx950.
//
// What the reference builds on the host, per step, from Python lists
// (slipstream/memory/paged_cache.py:71-109, build_paged_forward: seq_lens, query_lens
// and the flat slot_mapping of every new token) plus the packed description of the
// varlen kernel: from device-resident block tables, prior KV lengths and query
// lengths, one launch writes
//   cu_seqlens[b]   = sum of query_lens[i] for i < b        (cu_seqlens[B] = total)
//   context_lens[b] = prior_lens[b] + query_lens[b]         (seq_lens after the step)
//   slot_mapping[cu_seqlens[b] + j] = table[b][p / bs] * bs + p % bs,  p = prior_lens[b] + j
// which is the slot BlockManagerImpl.append_slot hands out for the token at position
// p when the table's earlier blocks are full (block_manager.py:141-159,282-287:
// tokens fill the first not-full block in table order). A position past the table or
// on a negative entry gets slot -1 (the scatter skips it), and so does every entry
// of slot_mapping past the step's last token. With this, a step's
// metadata needs no host lists, no uploads and no host synchronisation, so the step
// can be captured in a graph and replayed with new lengths.
//
// Work layout: workgroup b owns sequence b; its threads sum the query lengths of the
// sequences before it (one reduction, so no cross-workgroup pass is needed) and
// then write that sequence's slots, one token per thread.
#include "ss_common.h"

namespace {

struct MetaArgs {
  const int32_t* tables;
  int64_t bt_stride;
  int max_blocks;
  const int32_t* prior;
  const int32_t* qlens;
  int batch;
  int block_size;
  int bs_shift;
  int32_t* cu;
  int32_t* ctx;
  int64_t* slots;
  int64_t total;  // slot_mapping capacity
};

__global__ __launch_bounds__(256) void step_metadata_kernel(const MetaArgs a) {
  __shared__ int64_t s_part[4];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  int64_t part = 0;
  for (int i = tid; i < b; i += 256) part += max(a.qlens[i], 0);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) part += __shfl_xor(part, o);
  if ((tid & 63) == 0) s_part[tid >> 6] = part;
  __syncthreads();
  const int64_t base = s_part[0] + s_part[1] + s_part[2] + s_part[3];
  const int q = max(a.qlens[b], 0);
  const int p0 = max(a.prior[b], 0);
  if (tid == 0) {
    a.cu[b] = (int32_t)base;
    a.ctx[b] = p0 + q;
    if (b == a.batch - 1) a.cu[a.batch] = (int32_t)(base + q);
  }
  // a slot_mapping longer than the step's tokens: its tail must not hold stale slots,
  // which the scatter would take for real ones and write other sequences' pages
  if (b == a.batch - 1)
    for (int64_t t = base + q + tid; t < a.total; t += 256) a.slots[t] = -1;
  const int32_t* row = a.tables + (int64_t)b * a.bt_stride;
  for (int j = tid; j < q; j += 256) {
    const int64_t t = base + j;
    if (t >= a.total) break;
    const int64_t p = (int64_t)p0 + j;
    const int64_t bi = a.bs_shift >= 0 ? p >> a.bs_shift : p / a.block_size;
    const int64_t off = p - bi * a.block_size;
    const int32_t e = bi < a.max_blocks ? row[bi] : -1;
    a.slots[t] = e >= 0 ? (int64_t)e * a.block_size + off : -1;
  }
}

}  // namespace

extern "C" int ss_build_step_metadata(const int32_t* block_tables, int64_t bt_stride, int max_blocks,
                                      const int32_t* prior_lens, const int32_t* query_lens, int batch,
                                      int block_size, int32_t* cu_seqlens, int32_t* context_lens,
                                      int64_t* slot_mapping, int64_t total_tokens, void* stream) {
  const char* who = "build_step_metadata";
  if (batch < 0 || max_blocks < 0 || total_tokens < 0 || bt_stride < 0) {
    ss_host::set_error("%s: negative extent", who);
    return SS_ERR_INVALID;
  }
  if (block_size < 1) {
    ss_host::set_error("%s: block_size must be >= 1, got %d", who, block_size);
    return SS_ERR_INVALID;
  }
  if (batch == 0) return SS_OK;
  if (!block_tables || !prior_lens || !query_lens || !cu_seqlens || !context_lens ||
      (total_tokens > 0 && !slot_mapping)) {
    ss_host::set_error("%s: null pointer", who);
    return SS_ERR_INVALID;
  }
  MetaArgs a;
  a.tables = block_tables;
  a.bt_stride = bt_stride;
  a.max_blocks = max_blocks;
  a.prior = prior_lens;
  a.qlens = query_lens;
  a.batch = batch;
  a.block_size = block_size;
  a.bs_shift = ((block_size & (block_size - 1)) == 0) ? __builtin_ctz((unsigned)block_size) : -1;
  a.cu = cu_seqlens;
  a.ctx = context_lens;
  a.slots = slot_mapping;
  a.total = total_tokens;
  hipLaunchKernelGGL(step_metadata_kernel, dim3((unsigned)batch), dim3(256), 0, (hipStream_t)stream, a);
  return ss_host::launch_status(who);
}
