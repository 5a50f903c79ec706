// C-ABI entry points of paged attention: argument checks, then the split-K
// decode kernel for sequences whose query rows fit one 16-row MFMA tile, and
// the prefill kernel for the rest.
#include <algorithm>
#include <mutex>

#include "attention_common.h"

namespace ss {
int64_t decode_workspace_bytes(int dtype, int head_dim, int n_q, int n_kv, int max_query_len);
// plan_work / plan_qtiles: also build the tiled prefill's work list there (one more
// workgroup of the decode launch); *planned tells whether it did
int launch_decode(const AttnParams& p, int dtype, int head_dim, int max_query_len, char* ws,
                  int64_t ws_bytes, hipStream_t stream, int* plan_work = nullptr, int plan_qtiles = 0,
                  bool* planned = nullptr, DeferredMerge* defer = nullptr);
// the tiled prefill over a planned work list plus a deferred decode merge, one launch
int launch_prefill_merge(const AttnParams& pp, int dtype, int head_dim, int max_query_len, const int* work,
                         const DeferredMerge& dm, hipStream_t stream);
// shared-prefix cascade: prefix pass (pp, n_pf workgroups) and suffix decode (ps) in one
// launch, then the merge
int launch_cascade(const AttnParams& pp, const AttnParams& ps, int n_pf, int dtype, int head_dim, char* ws,
                   int64_t ws_bytes, hipStream_t stream);
int decode_heads_per_wg(int n_kv);
int64_t cascade_decode_bytes(int dtype, int head_dim, int n_kv, int rmax, int n_ranges);
int64_t prefill_work_bytes(int64_t batch, int n_rep, int max_query_len);
int64_t prefill_row_cap(int n_rep, int max_query_len);
// planned: work already holds the list (count, then (b << 16) | query tile per entry)
int launch_prefill(const AttnParams& p, int dtype, int head_dim, int max_query_len, int* work,
                   int64_t work_bytes, hipStream_t stream, bool planned);
int read_status(int* flags, int clear, hipStream_t stream);
int64_t general_workspace_bound(int n_q, int n_kv, int head_dim, int max_query_len);
int launch_general(const AttnParams& p, int dtype, int head_dim, int max_query_len, bool vec, void* ws,
                   int64_t ws_bytes, hipStream_t stream);
}  // namespace ss

namespace {

using ss::AttnParams;

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Shapes every entry point accepts: GQA, bf16 / fp16 / fp32, head_dim 1..256, any
// block size up to 1024 (the reference's Triton decode: head_dim <= 256, block_size
// <= 128, any float dtype; triton_paged.py:22-23,283-284).
int check_common(const char* who, int n_q, int n_kv, int head_dim, int block_size, int dtype,
                 int max_blocks, int64_t num_blocks) {
  if (n_kv < 1 || n_q < 1 || n_q % n_kv != 0) {
    ss_host::set_error("%s: GQA requires n_q %% n_kv == 0, got n_q=%d n_kv=%d", who, n_q, n_kv);
    return SS_ERR_INVALID;
  }
  if (dtype != SS_DTYPE_BF16 && dtype != SS_DTYPE_F16 && dtype != SS_DTYPE_F32) {
    ss_host::set_error("%s: dtype code %d not supported (bf16, fp16, fp32)", who, dtype);
    return SS_ERR_UNSUPPORTED;
  }
  if (head_dim < 1 || head_dim > 256) {
    ss_host::set_error("%s: head_dim %d not supported (1..256)", who, head_dim);
    return SS_ERR_UNSUPPORTED;
  }
  if (block_size < 1 || block_size > 1024) {
    ss_host::set_error("%s: block_size %d not supported (1..1024)", who, block_size);
    return SS_ERR_UNSUPPORTED;
  }
  if (max_blocks < 0 || num_blocks < 0) {
    ss_host::set_error("%s: negative table width or pool size", who);
    return SS_ERR_INVALID;
  }
  return SS_OK;
}

// dtype and head_dim of the MFMA kernels (bf16 / fp16, head_dim 64, 128 or 256).
bool mfma_dtype_dim(int dtype, int head_dim) {
  return (dtype == SS_DTYPE_BF16 || dtype == SS_DTYPE_F16) && (head_dim == 64 || head_dim == 128 || head_dim == 256);
}

bool strides_mult(const int64_t* s, int n, int64_t m) {
  for (int i = 0; i < n; ++i)
    if (s[i] % m != 0) return false;
  return true;
}

// Which kernels a call takes: the MFMA decode / prefill kernels when the dtype, head_dim,
// block size (a power of two, at least 4) and every 16-byte row condition allow, else the
// general kernel (paged_general.hip); vec: the general kernel may read the cache rows in
// 16-byte pieces.
struct Route {
  bool mfma;
  bool vec;
};

Route route(int dtype, int head_dim, int block_size, const void* q, const void* out, const void* k_cache,
            const void* v_cache, const int64_t* q_strides, int nq, const int64_t* o_strides, int no,
            const int64_t c_strides[3]) {
  const int elem = dtype == SS_DTYPE_F32 ? 4 : 2;
  const bool planes16 = aligned16(k_cache) && aligned16(v_cache) && strides_mult(c_strides, 3, 16 / elem) &&
                        ((int64_t)head_dim * elem) % 16 == 0;
  Route r;
  r.mfma = mfma_dtype_dim(dtype, head_dim) && block_size >= 4 && (block_size & (block_size - 1)) == 0 &&
           planes16 && strides_mult(q_strides, nq, 8) && strides_mult(o_strides, no, 8) && aligned16(q) &&
           aligned16(out);
  r.vec = planes16;
  return r;
}

void fill_common(AttnParams& p, const void* q, void* out, const void* k_cache, const void* v_cache,
                 const int32_t* block_tables, const int32_t* ctx_lens, int64_t batch, int n_q, int n_kv,
                 int max_blocks, int block_size, int64_t num_blocks, const int64_t c_strides[3],
                 int64_t bt_stride, float scale) {
  p.q = q;
  p.out = out;
  p.kc = k_cache;
  p.vc = v_cache;
  p.bt = block_tables;
  p.ctx_lens = ctx_lens;
  p.c_sb = c_strides[0];
  p.c_so = c_strides[1];
  p.c_sh = c_strides[2];
  p.bt_stride = bt_stride;
  p.num_blocks = num_blocks;
  p.batch = (int)batch;
  p.n_q = n_q;
  p.n_kv = n_kv;
  p.n_rep = n_q / n_kv;
  p.max_blocks = max_blocks;
  p.block_size = block_size;
  p.bs_shift = __builtin_ctz((unsigned)block_size);
  p.scale_log2 = scale * ss::kLog2e;
  p.total_tokens = 0x7fffffff;
  p.row_cap = 0;
}

// Workspace layout: [decode split-K partials, 256-byte aligned][prefill work list].
int64_t decode_part_bytes(int dtype, int head_dim, int n_q, int n_kv, int max_query_len) {
  return (ss::decode_workspace_bytes(dtype, head_dim, n_q, n_kv, max_query_len) + 255) & ~(int64_t)255;
}

int run(AttnParams& p, int dtype, int head_dim, int max_query_len, void* workspace, int64_t ws_bytes,
        hipStream_t stream, bool decode_rows, bool prefill_rows, const Route& rt) {
  // shapes outside the MFMA tiles: one general launch covers every row of the call
  if (!rt.mfma) return ss::launch_general(p, dtype, head_dim, max_query_len, rt.vec, workspace, ws_bytes, stream);
  p.rmax = ss::decode_rows_for(max_query_len, p.n_rep);
  p.row_cap = prefill_rows ? (int)std::min<int64_t>(ss::prefill_row_cap(p.n_rep, max_query_len), 0x7fffffff) : 0;
  const int64_t dec_bytes = decode_part_bytes(dtype, head_dim, p.n_q, p.n_kv, max_query_len);
  const bool has_list = workspace && ws_bytes > dec_bytes;
  int* const list = has_list ? (int*)((char*)workspace + dec_bytes) : nullptr;
  auto decode = [&](hipStream_t s, int* plan_work, int plan_qtiles, bool* planned, ss::DeferredMerge* defer) {
    return ss::launch_decode(p, dtype, head_dim, max_query_len, (char*)workspace, ws_bytes, s, plan_work,
                             plan_qtiles, planned, defer);
  };
  auto prefill = [&](hipStream_t s, bool planned) {
    return ss::launch_prefill(p, dtype, head_dim, max_query_len, list, has_list ? ws_bytes - dec_bytes : 0, s,
                              planned);
  };
  // A packed step has both kinds of rows. They run one after the other: each kernel
  // fills every CU with one workgroup (registers, LDS), and the split-K decode finishes
  // only when its last workgroup does, so sharing the GPU between them (a side stream)
  // made whichever started second trickle in behind the first. The decode goes first,
  // with one more workgroup that builds the tiled prefill's work list beside it (when
  // the prefill takes the tiled kernel: head_dim <= 128, blocks of >= 16 tokens); the
  // persistent prefill then takes all CUs for its balanced share.
  if (decode_rows && prefill_rows) {
    const int64_t qtiles = ((int64_t)std::max(max_query_len, 1) * p.n_rep + 127) / 128;
    // (the list's entries are (b << 16) | query tile: the limits the prefill launch checks)
    const bool tiled = head_dim <= 128 && p.block_size >= 16 && p.work_qtiles == 0 && list && qtiles <= 0xFFFF &&
                       p.batch <= 0x7FFF && (int64_t)p.batch * qtiles * p.n_kv <= 0x7fffffff &&
                       ws_bytes - dec_bytes >= ss::prefill_work_bytes(p.batch, p.n_rep, max_query_len);
    bool planned = false;
    ss::DeferredMerge dm{};
    // the decode's merge then runs in the tiled prefill's launch, on the CUs its
    // persistent workgroups leave as they finish
    int st = decode(stream, tiled ? list : nullptr, tiled ? (int)qtiles : 0, &planned, tiled ? &dm : nullptr);
    if (st != SS_OK) return st;
    // (the decode defers its merge only when it also built the list)
    if (dm.n_wg > 0) return ss::launch_prefill_merge(p, dtype, head_dim, max_query_len, list, dm, stream);
    return prefill(stream, planned);
  }
  if (decode_rows) return decode(stream, nullptr, 0, nullptr, nullptr);
  if (prefill_rows) return prefill(stream, false);
  return SS_OK;
}

}  // namespace

extern "C" int ss_paged_attention_workspace_size(int64_t batch, int n_q, int n_kv, int head_dim,
                                                 int max_query_len, int dtype, int64_t* bytes) {
  int st = check_common("paged attention workspace", n_q, n_kv, head_dim, 16, dtype, 0, 0);
  if (st != SS_OK) return st;
  if (!bytes) {
    ss_host::set_error("paged attention workspace: null output pointer");
    return SS_ERR_INVALID;
  }
  if (batch < 0) {
    ss_host::set_error("paged attention workspace: negative batch");
    return SS_ERR_INVALID;
  }
  const int mq = max_query_len < 1 ? 1 : max_query_len;
  // the block size and strides are not known here: cover the general kernel too
  const int64_t gen = ss::general_workspace_bound(n_q, n_kv, head_dim, mq);
  const int64_t mfma = mfma_dtype_dim(dtype, head_dim)
                           ? decode_part_bytes(dtype, head_dim, n_q, n_kv, mq) + ss::prefill_work_bytes(batch, n_q / n_kv, mq)
                           : 0;
  *bytes = mfma > gen ? mfma : gen;
  return SS_OK;
}

extern "C" int ss_paged_attention(const void* q, void* out, const void* k_cache, const void* v_cache,
                                  const int32_t* block_tables, const int32_t* seq_lens, int64_t batch,
                                  int n_q, int n_kv, int head_dim, int tq, int max_blocks, int block_size,
                                  int64_t num_blocks, const int64_t q_strides[3],
                                  const int64_t o_strides[3], const int64_t c_strides[3],
                                  int64_t bt_stride, float scale, int dtype, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
  const char* who = "paged attention";
  int st = check_common(who, n_q, n_kv, head_dim, block_size, dtype, max_blocks, num_blocks);
  if (st != SS_OK) return st;
  if (batch < 0 || tq < 0) {
    ss_host::set_error("%s: negative batch or query length", who);
    return SS_ERR_INVALID;
  }
  if (batch == 0 || tq == 0) return SS_OK;
  if (batch > 0x7fffffff) {
    ss_host::set_error("%s: batch %lld too large", who, (long long)batch);
    return SS_ERR_UNSUPPORTED;
  }
  if (!q || !out || !k_cache || !v_cache || !block_tables || !seq_lens) {
    ss_host::set_error("%s: null q, out, cache plane, block_tables or seq_lens", who);
    return SS_ERR_INVALID;
  }
  const Route rt = route(dtype, head_dim, block_size, q, out, k_cache, v_cache, q_strides, 3, o_strides, 3, c_strides);
  AttnParams p = {};
  fill_common(p, q, out, k_cache, v_cache, block_tables, seq_lens, batch, n_q, n_kv, max_blocks,
              block_size, num_blocks, c_strides, bt_stride, scale);
  p.cu = nullptr;
  p.tq = tq;
  p.q_sb = q_strides[0];
  p.q_sh = q_strides[1];
  p.q_st = q_strides[2];
  p.o_sb = o_strides[0];
  p.o_st = o_strides[1];
  p.o_sh = o_strides[2];
  const bool decode = (int64_t)tq * p.n_rep <= ss::kDecodeRows;
  return run(p, dtype, head_dim, tq, workspace, workspace_bytes, (hipStream_t)stream, decode, !decode, rt);
}

namespace {

int varlen_impl(const char* who, const void* q, void* out, const void* k_cache, const void* v_cache,
                const int32_t* block_tables, const int32_t* cu_seqlens, const int32_t* context_lens, int64_t batch,
                int64_t total_tokens, int n_q, int n_kv, int head_dim, int max_query_len, int max_blocks,
                int block_size, int64_t num_blocks, const int64_t q_strides[2], const int64_t o_strides[2],
                const int64_t c_strides[3], int64_t bt_stride, float scale, int dtype, void* workspace,
                int64_t workspace_bytes, void* stream) {
  int st = check_common(who, n_q, n_kv, head_dim, block_size, dtype, max_blocks, num_blocks);
  if (st != SS_OK) return st;
  if (batch < 0 || total_tokens < 0 || max_query_len < 0) {
    ss_host::set_error("%s: negative batch, token count or max_query_len", who);
    return SS_ERR_INVALID;
  }
  // max_query_len == 0 with tokens present breaks the caller's promise like any
  // other short max_query_len: the decode merge zero-fills such rows and flags them
  if (batch == 0 || total_tokens == 0) return SS_OK;
  if (batch > 0x7fffffff || total_tokens > 0x7fffffff) {
    ss_host::set_error("%s: batch %lld or token count %lld too large (int32 cu_seqlens)", who, (long long)batch,
                       (long long)total_tokens);
    return SS_ERR_UNSUPPORTED;
  }
  if (!q || !out || !k_cache || !v_cache || !block_tables || !cu_seqlens || !context_lens) {
    ss_host::set_error("%s: null q, out, cache plane, block_tables, cu_seqlens or context_lens", who);
    return SS_ERR_INVALID;
  }
  const Route rt = route(dtype, head_dim, block_size, q, out, k_cache, v_cache, q_strides, 2, o_strides, 2, c_strides);
  AttnParams p = {};
  fill_common(p, q, out, k_cache, v_cache, block_tables, context_lens, batch, n_q, n_kv, max_blocks,
              block_size, num_blocks, c_strides, bt_stride, scale);
  p.cu = cu_seqlens;
  p.total_tokens = (int)total_tokens;
  p.tq = 0;
  p.q_sb = 0;
  p.q_st = q_strides[0];
  p.q_sh = q_strides[1];
  p.o_sb = 0;
  p.o_st = o_strides[0];
  p.o_sh = o_strides[1];
  const bool prefill = (int64_t)max_query_len * p.n_rep > ss::kDecodeRows;
  return run(p, dtype, head_dim, max_query_len, workspace, workspace_bytes, (hipStream_t)stream, true,
             prefill, rt);
}

// Scratch of the no-alloc entry point: one array per GPU, held until the process
// ends. Host code never uses its name as an address (on the host it is a stand-in
// symbol); scratch_ptr() resolves this device's copy with hipGetSymbolAddress once
// per device, and only that pointer reaches the kernels.
constexpr int64_t kScratchBytes = 64ll << 20;
static __device__ __align__(256) char scratch[kScratchBytes];
std::mutex g_scratch_mutex;
void* g_scratch_ptr[64] = {nullptr};

void* scratch_ptr(const char* who) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    ss_host::set_error("%s: no current HIP device", who);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr) {
      ss_host::set_error("%s: hipGetSymbolAddress of the scratch array failed on device %d: %s", who, dev,
                         hipGetErrorString(err));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" int ss_paged_attention_varlen(const void* q, void* out, const void* k_cache, const void* v_cache,
                                         const int32_t* block_tables, const int32_t* cu_seqlens,
                                         const int32_t* context_lens, int64_t batch, int64_t total_tokens,
                                         int n_q, int n_kv, int head_dim, int max_query_len, int max_blocks,
                                         int block_size, int64_t num_blocks, const int64_t q_strides[2],
                                         const int64_t o_strides[2], const int64_t c_strides[3],
                                         int64_t bt_stride, float scale, int dtype, void* workspace,
                                         int64_t workspace_bytes, void* stream) {
  return varlen_impl("paged attention varlen", q, out, k_cache, v_cache, block_tables, cu_seqlens, context_lens,
                     batch, total_tokens, n_q, n_kv, head_dim, max_query_len, max_blocks, block_size, num_blocks,
                     q_strides, o_strides, c_strides, bt_stride, scale, dtype, workspace, workspace_bytes, stream);
}

extern "C" int ss_paged_attention_varlen_noalloc(const void* q, void* out, const void* k_cache, const void* v_cache,
                                                 const int32_t* block_tables, const int32_t* cu_seqlens,
                                                 const int32_t* context_lens, int64_t batch, int64_t total_tokens,
                                                 int n_q, int n_kv, int head_dim, int max_query_len, int max_blocks,
                                                 int block_size, int64_t num_blocks, const int64_t q_strides[2],
                                                 const int64_t o_strides[2], const int64_t c_strides[3],
                                                 int64_t bt_stride, float scale, int dtype, void* stream) {
  const char* who = "paged attention varlen (no-alloc)";
  // nothing to attend, or an argument error: the shared body returns without the scratch
  if (batch <= 0 || total_tokens <= 0 || n_q < 1 || n_kv < 1 || n_q % n_kv != 0)
    return varlen_impl(who, q, out, k_cache, v_cache, block_tables, cu_seqlens, context_lens, batch, total_tokens,
                       n_q, n_kv, head_dim, max_query_len, max_blocks, block_size, num_blocks, q_strides, o_strides,
                       c_strides, bt_stride, scale, dtype, nullptr, 0, stream);
  int64_t need = 0;
  int st = ss_paged_attention_workspace_size(batch, n_q, n_kv, head_dim, max_query_len < 1 ? 1 : max_query_len,
                                             dtype, &need);
  if (st != SS_OK) return st;
  if (need > kScratchBytes) {
    ss_host::set_error("%s: needs %lld bytes of scratch (batch %lld, max_query_len %d), the static scratch holds "
                       "%lld; use ss_paged_attention_varlen with a workspace", who, (long long)need,
                       (long long)batch, max_query_len, (long long)kScratchBytes);
    return SS_ERR_WORKSPACE;
  }
  void* ws = scratch_ptr(who);
  if (!ws) return SS_ERR_LAUNCH;
  return varlen_impl(who, q, out, k_cache, v_cache, block_tables, cu_seqlens, context_lens, batch, total_tokens,
                     n_q, n_kv, head_dim, max_query_len, max_blocks, block_size, num_blocks, q_strides, o_strides,
                     c_strides, bt_stride, scale, dtype, ws, kScratchBytes, stream);
}

// ---- shared-prefix cascade -------------------------------------------------
//
// A decode batch whose block tables all begin with the same prefix_blocks blocks
// (prefix-cache hits share full blocks) attends that prefix once for every
// sequence's query rows instead of once per sequence. One launch (cascade_kernel)
// runs parts 1 and 2 side by side on disjoint workgroups, the merge launch follows:
//   1. the prefix is cut into S chunks of cb blocks; chunk s is a pseudo-sequence
//      whose keys are the chunk (its table: entries s*cb .. of the first table row,
//      which holds the shared prefix) and whose queries are the whole batch's (read
//      in place, token t from row t % batch), without a causal mask. The tiled
//      prefill computes every (chunk, batch row) part, normalised, and its
//      log-sum-exp;
//   2. the decode attends each sequence's private suffix through its table from
//      column prefix_blocks on (KV length seq_len - prefix tokens), leaving fp32
//      partials; its merge completes every row, folding in the S prefix parts with
//      weights 2^(lse - max).
// Softmax over a union of disjoint key sets is the lse-weighted mix of the parts'
// softmaxes, so the result is the plain decode's up to rounding (the prefix parts
// are stored in the head_dim type, the suffix state stays fp32).

namespace {

struct PrefixPlan {
  bool cascade = false;
  int cb = 0, S = 0;
  int n_pf = 0, dec_ranges = 0;  // workgroups of the prefix pass; decode ranges per head group
  int64_t dec = 0, work = 0, lse = 0, part = 0, seq = 0;
  int64_t total() const { return dec + work + lse + part + seq; }
};

int64_t round256(int64_t x) { return (x + 255) & ~(int64_t)255; }

PrefixPlan prefix_plan(int64_t batch, int n_q, int n_kv, int head_dim, int block_size, int prefix_blocks,
                       int dtype) {
  PrefixPlan pl;
  const int n_rep = n_q / n_kv;
  if (!mfma_dtype_dim(dtype, head_dim)) {  // the general kernel, one query token per sequence
    pl.dec = ss::general_workspace_bound(n_q, n_kv, head_dim, 1);
    return pl;
  }
  pl.dec = decode_part_bytes(dtype, head_dim, n_q, n_kv, 1);
  // the prefill's tiled kernel (head_dim <= 128, blocks of 16+ tokens) carries the
  // prefix pass and the decode kernel the suffixes (n_rep <= 16); other shapes, and
  // batches whose rows fit one decode tile, take the plain path of one query token
  pl.cascade = prefix_blocks > 0 && head_dim <= 128 && block_size >= 16 && n_rep <= ss::kDecodeRows &&
               batch * n_rep > ss::kDecodeRows;
  if (!pl.cascade) {
    pl.work = ss::prefill_work_bytes(batch, n_rep, 1);
    return pl;
  }
  // The prefix pass and the suffix decode run in one launch on disjoint CUs: 3/8 of
  // them take the prefix chunks (about one item each: items = S * row tiles * n_kv;
  // chunks hold whole 64-key tiles) and the rest the decode ranges. C4 (256 CUs, 28
  // items per chunk), whole call in a graph: S = 2 / 3 / 4 / 5 (56 / 84 / 112 / 140
  // prefix workgroups) 34.4 / 29.3 / 29.6 / 33.2 us.
  const int64_t per_chunk = ((batch * n_rep + 127) / 128) * n_kv;
  const int64_t cus = ss_host::device_cu_count();
  int64_t px_wgs = cus * 3 / 8;
  if (px_wgs < 1) px_wgs = 1;
  int64_t target = px_wgs / per_chunk;
  if (target < 1) target = 1;
  const int tile_blocks = 64 / block_size > 1 ? 64 / block_size : 1;
  int64_t cb = (prefix_blocks + target - 1) / target;
  cb = (cb + tile_blocks - 1) / tile_blocks * tile_blocks;
  // a chunk never outgrows the prefix: the chunk tables (entries s*cb .. s*cb + cb - 1
  // of the first row, s < S) then stay below prefix_blocks + cb <= 2 * max_blocks
  // entries, inside the table of a batch of two or more rows
  if (cb > prefix_blocks) cb = prefix_blocks;
  pl.cb = (int)cb;
  pl.S = (int)((prefix_blocks + cb - 1) / cb);
  const int64_t items = pl.S * per_chunk;
  pl.n_pf = (int)(items < px_wgs ? items : px_wgs);
  // two decode ranges per workgroup (one per half of its eight waves)
  const int64_t hgroups = n_kv / ss::decode_heads_per_wg(n_kv);
  const int64_t rest = (cus - pl.n_pf) / hgroups;
  pl.dec_ranges = 2 * (int)(rest > 1 ? rest : 1);
  pl.dec = round256(ss::cascade_decode_bytes(dtype, head_dim, n_kv, ss::decode_rows_for(1, n_rep), pl.dec_ranges));
  const int64_t elem = 2;  // bf16 / fp16
  pl.work = 0;  // the prefix pass walks its (chunk, query tile) items in order
  pl.lse = round256(4 * (int64_t)pl.S * batch * n_q);
  pl.part = round256((int64_t)pl.S * batch * n_q * head_dim * elem);
  pl.seq = round256(batch * n_q * (int64_t)(head_dim + 2) * 4);  // fp32 rows of suffixes finished in one range
  return pl;
}

}  // namespace

extern "C" int ss_paged_attention_shared_prefix_workspace_size(int64_t batch, int n_q, int n_kv, int head_dim,
                                                               int block_size, int prefix_blocks, int dtype,
                                                               int64_t* bytes) {
  const char* who = "shared-prefix attention workspace";
  int st = check_common(who, n_q, n_kv, head_dim, block_size, dtype, 0, 0);
  if (st != SS_OK) return st;
  if (!bytes) {
    ss_host::set_error("%s: null output pointer", who);
    return SS_ERR_INVALID;
  }
  if (batch < 0 || prefix_blocks < 0) {
    ss_host::set_error("%s: negative batch or prefix_blocks", who);
    return SS_ERR_INVALID;
  }
  *bytes = prefix_plan(batch, n_q, n_kv, head_dim, block_size, prefix_blocks, dtype).total();
  return SS_OK;
}

extern "C" int ss_paged_attention_shared_prefix(const void* q, void* out, const void* k_cache, const void* v_cache,
                                                const int32_t* block_tables, const int32_t* seq_lens, int64_t batch,
                                                int n_q, int n_kv, int head_dim, int max_blocks, int block_size,
                                                int64_t num_blocks, int prefix_blocks, const int64_t q_strides[2],
                                                const int64_t o_strides[2], const int64_t c_strides[3],
                                                int64_t bt_stride, float scale, int dtype, void* workspace,
                                                int64_t workspace_bytes, void* stream) {
  const char* who = "shared-prefix attention";
  int st = check_common(who, n_q, n_kv, head_dim, block_size, dtype, max_blocks, num_blocks);
  if (st != SS_OK) return st;
  if (batch < 0 || prefix_blocks < 0 || prefix_blocks > max_blocks) {
    ss_host::set_error("%s: need batch >= 0 and 0 <= prefix_blocks <= max_blocks (got %lld, %d, %d)", who,
                       (long long)batch, prefix_blocks, max_blocks);
    return SS_ERR_INVALID;
  }
  if (batch == 0) return SS_OK;
  if (batch > 0x7FFFFF) {
    ss_host::set_error("%s: batch %lld too large", who, (long long)batch);
    return SS_ERR_UNSUPPORTED;
  }
  if (!q || !out || !k_cache || !v_cache || !block_tables || !seq_lens) {
    ss_host::set_error("%s: null q, out, cache plane, block_tables or seq_lens", who);
    return SS_ERR_INVALID;
  }
  const Route rt = route(dtype, head_dim, block_size, q, out, k_cache, v_cache, q_strides, 2, o_strides, 2, c_strides);
  const PrefixPlan pl = prefix_plan(batch, n_q, n_kv, head_dim, block_size, prefix_blocks, dtype);
  if (!workspace || workspace_bytes < pl.total()) {
    ss_host::set_error("%s: workspace of %lld bytes, needs %lld", who, (long long)workspace_bytes,
                       (long long)pl.total());
    return SS_ERR_WORKSPACE;
  }
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  AttnParams p = {};
  fill_common(p, q, out, k_cache, v_cache, block_tables, seq_lens, batch, n_q, n_kv, max_blocks, block_size,
              num_blocks, c_strides, bt_stride, scale);
  p.cu = nullptr;
  p.tq = 1;
  p.q_sb = q_strides[0];
  p.q_sh = q_strides[1];
  p.q_st = 0;
  p.o_sb = o_strides[0];
  p.o_sh = o_strides[1];
  p.o_st = 0;
  if (!pl.cascade || !rt.mfma) {
    const bool dec = p.n_rep <= ss::kDecodeRows;
    return run(p, dtype, head_dim, 1, ws, pl.dec + pl.work, s, dec, !dec, rt);
  }

  float* lse = (float*)(ws + pl.dec + pl.work);
  void* part = ws + pl.dec + pl.work + pl.lse;
  float* seq_o = (float*)(ws + pl.dec + pl.work + pl.lse + pl.part);
  float* seq_ml = seq_o + batch * n_q * (int64_t)head_dim;
  const int64_t qtiles = (batch * p.n_rep + 127) / 128;
  if (qtiles > 0xFFFF || pl.S > 0x7FFF || pl.S * qtiles * n_kv > 0x7fffffff) {
    ss_host::set_error("%s: too many query tiles for the prefix pass (%lld per chunk, %d chunks)", who,
                       (long long)qtiles, pl.S);
    return SS_ERR_UNSUPPORTED;
  }
  // 1. prefix chunks as pseudo-sequences of the tiled prefill, queries read in place
  AttnParams pp = {};
  fill_common(pp, q, part, k_cache, v_cache, block_tables, nullptr, pl.S, n_q, n_kv, pl.cb, block_size, num_blocks,
              c_strides, pl.cb, scale);
  pp.chunk_tokens = pl.cb * block_size;
  pp.prefix_tokens = prefix_blocks * block_size;
  pp.work_qtiles = (int)qtiles;
  pp.q_sb = 0;
  pp.q_st = q_strides[0];
  pp.q_sh = q_strides[1];
  pp.o_sb = 0;
  pp.o_st = (int64_t)n_q * head_dim;
  pp.o_sh = head_dim;
  pp.rmax = ss::decode_rows_for((int)batch, pp.n_rep);
  pp.lse = lse;
  pp.noncausal = 1;
  pp.q_period = (int)batch;
  // 2. private suffixes: the table from column prefix_blocks on, lengths past the
  // prefix; the prefix parts are folded in where each row is finished
  AttnParams ps = p;
  ps.bt = block_tables + prefix_blocks;
  ps.max_blocks = max_blocks - prefix_blocks;
  ps.ctx_shift = prefix_blocks * block_size;
  ps.rmax = ss::decode_rows_for(1, ps.n_rep);
  ps.px_part = part;
  ps.px_lse = lse;
  ps.px_n = pl.S;
  ps.px_seq_o = seq_o;
  ps.px_seq_ml = seq_ml;
  ps.range_cap = pl.dec_ranges;
  return ss::launch_cascade(pp, ps, pl.n_pf, dtype, head_dim, ws, pl.dec, s);
}

extern "C" int ss_attention_status(int* flags, int clear, void* stream) {
  if (!flags) {
    ss_host::set_error("attention status: null output pointer");
    return SS_ERR_INVALID;
  }
  const int st = ss::read_status(flags, clear, (hipStream_t)stream);
  if (st != SS_OK) ss_host::set_error("attention status: %s", hipGetErrorString(hipGetLastError()));
  return st;
}
