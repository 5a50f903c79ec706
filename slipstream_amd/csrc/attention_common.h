// Parameters and per-sequence metadata shared by the paged-attention kernels.
#pragma once

#include "ss_common.h"

namespace ss {

// Everything a paged-attention launch needs. Pointers are raw device pointers,
// strides are in elements. A sequence ("row" of the batch) b owns query tokens
// [qoff(b), qoff(b) + qlen(b)) and ctx(b) KV tokens reached through
// block_tables[b * bt_stride + i].
struct AttnParams {
  const void* q;
  void* out;
  const void* kc;  // K plane of the layer: [num_blocks, block_size, n_kv, D]
  const void* vc;  // V plane of the layer, same strides
  const int32_t* bt;
  const int32_t* ctx_lens;  // seq_lens / context_lens [batch]
  const int32_t* cu;        // cu_seqlens [batch+1] for the packed form, nullptr when padded
  int64_t q_sb, q_st, q_sh;  // padded: (b, t, h); packed: q_sb = 0, q_st = token stride
  int64_t o_sb, o_st, o_sh;
  int64_t c_sb, c_so, c_sh;  // cache strides (block, offset, head)
  int64_t bt_stride;
  int64_t num_blocks;
  int batch, n_q, n_kv, n_rep;
  int tq;  // padded query length (unused when cu != nullptr)
  int max_blocks, bs_shift, block_size;
  float scale_log2;  // softmax scale * log2(e)
  // split-K decode bookkeeping (workspace carve-up)
  float* ws_o;   // [n_wg * 2 * hpw * rmax * D] unnormalised partial outputs
  float* ws_ml;  // [n_wg * 2 * hpw * rmax * 2]   (running max, running sum)
  int* ws_rec;   // [n_wg * 8] per-workgroup record of the split sequence it owns
  int n_ranges;          // work ranges of the decode stream-K partition
  int hpw;               // KV heads per decode workgroup (one wave each)
  int n_hgroups;         // n_kv / hpw
  int rmax;              // query rows per (sequence, KV head) stored in a partial
  // Shared-prefix cascade (zero / nullptr for plain attention):
  float* lse;     // when set, log2-domain log-sum-exp of each query row: [tokens, n_q]
  int noncausal;  // every query row sees all of its sequence's keys
  int q_period;   // when > 0, query token t is read from row t % q_period
  int range_cap;  // when > 0, at most this many decode ranges per head group
  // Packed form only: query tokens in q/out. cu_seqlens entries are clamped into
  // [0, total_tokens], so a stream description that runs past q never indexes
  // outside it.
  int total_tokens;
  // Query rows per (sequence, KV head) the prefill launch of this call covers
  // (query tiles x rows per tile; 0 when no prefill runs). Rows of a longer
  // sequence (a query longer than the call's max_query_len) are written as zeros
  // by the decode merge, which also raises kStatusQueryTooLong.
  int row_cap;
  // Shared-prefix cascade (zero / nullptr otherwise):
  int ctx_shift;      // KV length of sequence b = ctx_lens[b] - ctx_shift (at least 0)
  int chunk_tokens;   // > 0: sequence b is chunk b of a prefix of prefix_tokens keys:
  int prefix_tokens;  //   min(chunk_tokens, prefix_tokens - b * chunk_tokens) keys, no
                      //   ctx_lens, and query tokens [b * q_period, (b + 1) * q_period)
  int work_qtiles;    // > 0: the prefill takes entry e = (e / work_qtiles, e % work_qtiles)
                      //   of batch * work_qtiles, in order, instead of a work list
  const void* px_part;  // S normalised prefix parts [S][batch * n_q][D] of the head_dim type
  const float* px_lse;  // and their log2-domain log-sum-exp [S][batch * n_q]
  int px_n;             // S: the decode and its merge fold the parts into every row
  float* px_seq_o;      // fp32 (acc, then max and sum) of the rows of sequences the decode
  float* px_seq_ml;     //   finishes inside one range: [batch * n_q][D], [batch * n_q][2]
};

// Bits of the device status word (ss_attention_status): set by kernels that met a
// packed description they could not compute, never cleared by them.
constexpr int kStatusQueryTooLong = 1;   // qlen > max_query_len: rows zero-filled
constexpr int kStatusStreamOverrun = 2;  // cu_seqlens beyond total_tokens: clamped
constexpr int kStatusPrefixShort = 4;    // shared prefix longer than a sequence's seq_len

// Decode tile: one wave covers up to 16 query rows (query token j, head i in
// the GQA group) of one KV head; r = j * n_rep + i.
constexpr int kDecodeRows = 16;
// Keys per decode iteration: two 16-token MFMA tiles.
constexpr int kPairTokens = 32;

// cu_seqlens and context_lens are read through the constant address space: where the
// sequence index is wave-uniform that makes them scalar loads, whose waits (lgkmcnt)
// leave the vector loads in flight alone -- a vector load of them inside the decode's
// pipelined loop came with a wait for every K/V load in flight.
typedef const __attribute__((address_space(4))) int32_t* ConstI32;

__device__ __forceinline__ void seq_queries(const AttnParams& p, int b, int& qlen, int64_t& qoff) {
  if (p.chunk_tokens > 0) {
    qlen = p.q_period;
    qoff = (int64_t)b * p.q_period;
  } else if (p.cu) {
    const ConstI32 cu = (ConstI32)p.cu;
    const int s = min(max(cu[b], 0), p.total_tokens);
    const int e = min(max(cu[b + 1], s), p.total_tokens);
    qlen = e - s;
    qoff = s;
  } else {
    qlen = p.tq;
    qoff = 0;
  }
}

// Index of a query row's log-sum-exp: packed (or prefix-chunk) token, else b * tq + t,
// times n_q, plus head.
__device__ __forceinline__ int64_t lse_index(const AttnParams& p, int b, int64_t qoff, int j, int hq) {
  const int64_t tok = (p.cu || p.chunk_tokens > 0) ? qoff + j : (int64_t)b * p.tq + j;
  return tok * p.n_q + hq;
}

// KV length of sequence b (context_lens / seq_lens, negative counts as 0).
__device__ __forceinline__ int kv_len(const AttnParams& p, int b) {
  if (p.chunk_tokens > 0) return min(p.chunk_tokens, p.prefix_tokens - b * p.chunk_tokens);
  const int c = ((ConstI32)p.ctx_lens)[b] - p.ctx_shift;
  return c < 0 ? 0 : c;
}

// KV tokens reachable through the table (Triton: n_blocks = min(cdiv(len, bs), max_blocks)).
__device__ __forceinline__ int seq_kv_tokens(const AttnParams& p, int ctx) {
  const int cap = p.max_blocks << p.bs_shift;
  ctx = ctx < 0 ? 0 : ctx;
  return ctx < cap ? ctx : cap;
}

// Sequences whose qlen * n_rep query rows fit the decode tile (p.rmax <= 16 rows,
// set per launch from max_query_len) take the split-K decode kernel; the rest
// take the prefill kernel. Both kernels use this one predicate.
__device__ __forceinline__ bool is_decode_seq(const AttnParams& p, int qlen) {
  return qlen >= 1 && qlen * p.n_rep <= p.rmax;
}

// A decode launch's merge left to the next launch of the same call: the params it
// runs with (the decode's workspace carved in) and the decode's workgroup count.
struct DeferredMerge {
  AttnParams p;
  int n_wg;  // 0: nothing deferred
};

// Work list of the tiled prefill, built by one workgroup (blockDim.x a multiple of 64
// that divides kPlanBuckets): work[0] = entries, work[1 + i] = (b << 16) | qt for every
// (sequence, 128-row query tile) of a prefill sequence, ordered by decreasing cost
// (64-key tiles below the tile's causal end, plus one): a counting sort over cost
// buckets in LDS. Entries of equal cost land in any order; an item's result does not
// depend on the workgroup that computes it.
constexpr int kPlanBuckets = 1024;
__device__ __forceinline__ void plan_work_list(const AttnParams& p, int* __restrict__ work, int qtiles) {
  __shared__ int s_hist[kPlanBuckets];
  __shared__ int s_base[kPlanBuckets];
  __shared__ int s_wsum[kPlanBuckets / 64];
  const int tid = threadIdx.x, nt = blockDim.x;
  for (int c = tid; c < kPlanBuckets; c += nt) s_hist[c] = 0;
  __syncthreads();
  const int64_t n_entries = (int64_t)p.batch * qtiles;
  // cost bucket of entry e = b * qtiles + qt, or -1 when it is not a prefill tile
  auto bucket = [&](int64_t e) {
    const int b = (int)(e / qtiles), qt = (int)(e - (int64_t)b * qtiles);
    int qlen;
    int64_t qoff;
    seq_queries(p, b, qlen, qoff);
    if (qlen <= 0 || is_decode_seq(p, qlen)) return -1;
    const int R = qlen * p.n_rep, row0 = qt * 128;
    if (row0 >= R) return -1;
    const int ctx = kv_len(p, b);
    const int kvt = seq_kv_tokens(p, ctx);
    const int last_row = min(R - 1, row0 + 127);
    const int kv_end = p.noncausal ? kvt : min(kvt, ctx - qlen + last_row / p.n_rep + 1);
    const int cost = (kv_end > 0 ? (kv_end + 63) / 64 : 0) + 1;
    return min(cost, kPlanBuckets - 1);
  };
  for (int64_t e = tid; e < n_entries; e += nt) {
    const int c = bucket(e);
    if (c >= 0) atomicAdd(&s_hist[c], 1);
  }
  __syncthreads();
  {  // exclusive scan from the costliest bucket down: thread t takes the per = 1024 / nt
     // buckets 1023 - (per t + j), j < per
    const int per = kPlanBuckets / nt;
    const int lane = tid & 63, wave = tid >> 6;
    int sum = 0;
    for (int j = 0; j < per; ++j) sum += s_hist[kPlanBuckets - 1 - (per * tid + j)];
    int v = sum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_up(v, o);
      v += lane >= o ? t : 0;
    }
    if (lane == 63) s_wsum[wave] = v;
    __syncthreads();
    for (int w = 0; w < wave; ++w) v += s_wsum[w];
    int run = v - sum;
    for (int j = 0; j < per; ++j) {
      const int c = kPlanBuckets - 1 - (per * tid + j);
      s_base[c] = run;
      run += s_hist[c];
    }
    if (tid == nt - 1) work[0] = v;
  }
  __syncthreads();
  for (int64_t e = tid; e < n_entries; e += nt) {
    const int c = bucket(e);
    if (c >= 0) {
      const int b = (int)(e / qtiles), qt = (int)(e - (int64_t)b * qtiles);
      work[1 + atomicAdd(&s_base[c], 1)] = (b << 16) | qt;
    }
  }
}

// rmax for a launch whose longest query is max_query_len.
inline int decode_rows_for(int max_query_len, int n_rep) {
  long long r = (long long)(max_query_len < 1 ? 1 : max_query_len) * n_rep;
  return r > kDecodeRows ? kDecodeRows : (int)r;
}

}  // namespace ss
