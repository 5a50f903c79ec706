// C-ABI entry points of paged attention: argument checks, then the split-K
// decode kernel for sequences whose query rows fit one 16-row MFMA tile, and
// the prefill kernel for the rest.
#include "attention_common.h"

namespace ss {
int64_t decode_workspace_bytes(int dtype, int head_dim, int n_q, int n_kv, int max_query_len);
int launch_decode(const AttnParams& p, int dtype, int head_dim, int max_query_len, char* ws,
                  int64_t ws_bytes, hipStream_t stream);
int64_t prefill_work_bytes(int64_t batch, int n_rep, int max_query_len);
int launch_prefill(const AttnParams& p, int dtype, int head_dim, int max_query_len, int* work,
                   int64_t work_bytes, hipStream_t stream);
}  // namespace ss

namespace {

using ss::AttnParams;

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_common(const char* who, int n_q, int n_kv, int head_dim, int block_size, int dtype,
                 int max_blocks, int64_t num_blocks) {
  if (n_kv < 1 || n_q < 1 || n_q % n_kv != 0) {
    ss_host::set_error("%s: GQA requires n_q %% n_kv == 0, got n_q=%d n_kv=%d", who, n_q, n_kv);
    return SS_ERR_INVALID;
  }
  if (dtype != SS_DTYPE_BF16 && dtype != SS_DTYPE_F16) {
    ss_host::set_error("%s: dtype code %d not supported (bf16 and fp16 only)", who, dtype);
    return SS_ERR_UNSUPPORTED;
  }
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) {
    ss_host::set_error("%s: head_dim %d not supported (64, 128, 256)", who, head_dim);
    return SS_ERR_UNSUPPORTED;
  }
  if (block_size < 4 || block_size > 1024 || (block_size & (block_size - 1)) != 0) {
    ss_host::set_error("%s: block_size %d not supported (power of two, 4..1024)", who, block_size);
    return SS_ERR_UNSUPPORTED;
  }
  if (max_blocks < 0 || num_blocks < 0) {
    ss_host::set_error("%s: negative table width or pool size", who);
    return SS_ERR_INVALID;
  }
  return SS_OK;
}

int check_strides(const char* who, const int64_t* s, int n) {
  for (int i = 0; i < n; ++i) {
    if (s[i] % 8 != 0) {
      ss_host::set_error("%s: stride %lld is not a multiple of 8 elements (16-byte rows required)", who,
                         (long long)s[i]);
      return SS_ERR_UNSUPPORTED;
    }
  }
  return SS_OK;
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
}

// Workspace layout: [decode split-K partials, 256-byte aligned][prefill work list].
int64_t decode_part_bytes(int dtype, int head_dim, int n_q, int n_kv, int max_query_len) {
  return (ss::decode_workspace_bytes(dtype, head_dim, n_q, n_kv, max_query_len) + 255) & ~(int64_t)255;
}

int run(AttnParams& p, int dtype, int head_dim, int max_query_len, void* workspace, int64_t ws_bytes,
        hipStream_t stream, bool decode_rows, bool prefill_rows) {
  p.rmax = ss::decode_rows_for(max_query_len, p.n_rep);
  const int64_t dec_bytes = decode_part_bytes(dtype, head_dim, p.n_q, p.n_kv, max_query_len);
  auto decode = [&](hipStream_t s) {
    return ss::launch_decode(p, dtype, head_dim, max_query_len, (char*)workspace, ws_bytes, s);
  };
  auto prefill = [&](hipStream_t s) {
    const bool has_list = workspace && ws_bytes > dec_bytes;
    return ss::launch_prefill(p, dtype, head_dim, max_query_len, has_list ? (int*)((char*)workspace + dec_bytes) : nullptr,
                              has_list ? ws_bytes - dec_bytes : 0, s);
  };
  // A packed step has both kinds of rows. They run one after the other, the prefill
  // first: each kernel fills every CU with one workgroup (registers, LDS), and the
  // split-K decode finishes only when its last workgroup does, so sharing the GPU
  // between them (a side stream) made whichever started second trickle in behind
  // the first. The persistent prefill takes all CUs for its balanced share, then the
  // decode gets all CUs at once.
  if (decode_rows && prefill_rows) {
    int st = prefill(stream);
    return st != SS_OK ? st : decode(stream);
  }
  if (decode_rows) return decode(stream);
  if (prefill_rows) return prefill(stream);
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
  *bytes = decode_part_bytes(dtype, head_dim, n_q, n_kv, mq) + ss::prefill_work_bytes(batch, n_q / n_kv, mq);
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
  if ((st = check_strides(who, q_strides, 3)) != SS_OK) return st;
  if ((st = check_strides(who, o_strides, 3)) != SS_OK) return st;
  if ((st = check_strides(who, c_strides, 3)) != SS_OK) return st;
  if (!aligned16(q) || !aligned16(out) || !aligned16(k_cache) || !aligned16(v_cache)) {
    ss_host::set_error("%s: q, out and cache planes must be 16-byte aligned", who);
    return SS_ERR_UNSUPPORTED;
  }
  if (!block_tables || !seq_lens) {
    ss_host::set_error("%s: null block_tables or seq_lens", who);
    return SS_ERR_INVALID;
  }
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
  return run(p, dtype, head_dim, tq, workspace, workspace_bytes, (hipStream_t)stream, decode, !decode);
}

extern "C" int ss_paged_attention_varlen(const void* q, void* out, const void* k_cache, const void* v_cache,
                                         const int32_t* block_tables, const int32_t* cu_seqlens,
                                         const int32_t* context_lens, int64_t batch, int64_t total_tokens,
                                         int n_q, int n_kv, int head_dim, int max_query_len, int max_blocks,
                                         int block_size, int64_t num_blocks, const int64_t q_strides[2],
                                         const int64_t o_strides[2], const int64_t c_strides[3],
                                         int64_t bt_stride, float scale, int dtype, void* workspace,
                                         int64_t workspace_bytes, void* stream) {
  const char* who = "paged attention varlen";
  int st = check_common(who, n_q, n_kv, head_dim, block_size, dtype, max_blocks, num_blocks);
  if (st != SS_OK) return st;
  if (batch < 0 || total_tokens < 0 || max_query_len < 0) {
    ss_host::set_error("%s: negative batch, token count or max_query_len", who);
    return SS_ERR_INVALID;
  }
  if (batch == 0 || total_tokens == 0 || max_query_len == 0) return SS_OK;
  if (batch > 0x7fffffff) {
    ss_host::set_error("%s: batch %lld too large", who, (long long)batch);
    return SS_ERR_UNSUPPORTED;
  }
  if ((st = check_strides(who, q_strides, 2)) != SS_OK) return st;
  if ((st = check_strides(who, o_strides, 2)) != SS_OK) return st;
  if ((st = check_strides(who, c_strides, 3)) != SS_OK) return st;
  if (!aligned16(q) || !aligned16(out) || !aligned16(k_cache) || !aligned16(v_cache)) {
    ss_host::set_error("%s: q, out and cache planes must be 16-byte aligned", who);
    return SS_ERR_UNSUPPORTED;
  }
  if (!block_tables || !cu_seqlens || !context_lens) {
    ss_host::set_error("%s: null block_tables, cu_seqlens or context_lens", who);
    return SS_ERR_INVALID;
  }
  AttnParams p = {};
  fill_common(p, q, out, k_cache, v_cache, block_tables, context_lens, batch, n_q, n_kv, max_blocks,
              block_size, num_blocks, c_strides, bt_stride, scale);
  p.cu = cu_seqlens;
  p.tq = 0;
  p.q_sb = 0;
  p.q_st = q_strides[0];
  p.q_sh = q_strides[1];
  p.o_sb = 0;
  p.o_st = o_strides[0];
  p.o_sh = o_strides[1];
  const bool prefill = (int64_t)max_query_len * p.n_rep > ss::kDecodeRows;
  return run(p, dtype, head_dim, max_query_len, workspace, workspace_bytes, (hipStream_t)stream, true,
             prefill);
}
