// General paged attention for the shapes outside the MFMA kernels' tiles: fp32
// caches, any head_dim up to 256 (80, 96, 112, 8, ...), any block size, and element
// strides without 16-byte alignment.
//
// Math: the same as paged_decode.hip and paged_prefill.hip --
// slipstream/models/layers/attention.py:64-88 via attention_ref.py:68-89, the causal
// rule of attention.py:46-48 (query j of a Tq-token chunk sees keys
// [0, seq_len - Tq + j]) and the edge rules of triton_paged.py:133-206 (absent
// blocks masked, a row with no visible key is zero). The reference's Triton decode
// serves this whole range (triton_paged.py:22-23,283-284: head_dim <= 256,
// block_size <= 128, any float dtype), and its own parity test runs fp32 at
// head_dim 8 (tests/kernels/test_paged_attention.py:46-70).
//
// One workgroup = (sequence b, KV head h, tile of RT query rows, key split s). The
// rows are r = j * n_rep + i (query token j, head i of the GQA group), so the n_rep
// query heads of a KV head share every K/V row read. Four waves take the tile's
// 64-key blocks in turn (wave w: blocks w, w + 4, ...). Per block:
//   scores: lane = key. The lane reads its key's K row (16-byte loads when the row
//           and strides allow, else element loads) and forms RT dot products against
//           the query rows held in LDS as fp32, pre-scaled by scale * log2(e) (every
//           lane reads the same LDS address: broadcasts);
//   online softmax in fp32 (exp2 domain), each row's max over the wave's 64 keys;
//   P goes to the wave's LDS slice, then O += P V with lane = d (d = lane + 64 c),
//           so every V row read is one coalesced row.
// The waves merge through LDS in a fixed order (deterministic). With one key split
// the workgroup writes the output rows; with several it writes fp32 partials (max,
// sum, unnormalised output) that general_merge_kernel combines in split order.
// Arithmetic is fp32 throughout (fp32 softmax as in attention.py:82), the output is
// rounded once to the query's type.
#include "attention_common.h"

namespace ss {
namespace {

constexpr int kGenWaves = 4;
constexpr int kGenKeys = 64;      // keys per wave block: one per lane
constexpr int kGenMaxDim = 256;   // head_dim bound (triton_paged.py:22)
constexpr int kGenMaxSplits = 16;

// Target of the loads of absent keys (masked; never written, so zero).
__device__ __attribute__((aligned(16))) float g_gen_zero[kGenMaxDim];

// Status bits raised by this file's kernels (kStatus* of attention_common.h); read
// and cleared together with the decode's word by ss_attention_status.
__device__ int g_gen_status;
__device__ int g_gen_status_seen;

__global__ void gen_status_take_kernel(int clear) {
  g_gen_status_seen = clear ? atomicExch(&g_gen_status, 0) : atomicOr(&g_gen_status, 0);
}

struct GenArgs {
  int head_dim;
  int qst;       // LDS row stride of the query and output slabs (floats, head_dim rounded to 4)
  int tiles;     // row tiles per (sequence, KV head)
  int ksplit;    // key splits per row tile
  float* part_o;   // ksplit > 1: [units * ksplit * RT][head_dim] unnormalised outputs
  float* part_ml;  //   and [units * ksplit * RT][2] (max, sum), log2 domain
};

template <typename T>
__device__ __forceinline__ float to_f32(T x) {
  return (float)x;
}

// The 16 / sizeof(T) elements of a 16-byte chunk, widened to fp32.
template <typename T>
__device__ __forceinline__ void widen16(u32x4 v, float* f) {
  if constexpr (sizeof(T) == 4) {
    // through a scalar: __builtin_bit_cast of a vector element v[e] reads element 0
    // for every e with this compiler
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t w = v[e];
      f[e] = __builtin_bit_cast(float, w);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[2 * e] = Elem<T>::lo(v[e]);
      f[2 * e + 1] = Elem<T>::hi(v[e]);
    }
  }
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// KV tokens of a length-ctx sequence reachable through a table of max_blocks entries.
__device__ __forceinline__ int gen_kv_tokens(const AttnParams& p, int ctx) {
  const int64_t cap = (int64_t)p.max_blocks * p.block_size;
  ctx = ctx < 0 ? 0 : ctx;
  return (int64_t)ctx < cap ? ctx : (int)cap;
}

// Decomposes the grid index: unit = (b, h, tile), then the key split.
struct GenWork {
  int b, h, tile, split;
  int64_t unit;
};

__device__ __forceinline__ GenWork gen_work(const AttnParams& p, const GenArgs& g, int64_t blk) {
  GenWork w;
  w.split = (int)(blk % g.ksplit);
  w.unit = blk / g.ksplit;
  w.tile = (int)(w.unit % g.tiles);
  const int64_t bh = w.unit / g.tiles;
  w.h = (int)(bh % p.n_kv);
  w.b = (int)(bh / p.n_kv);
  return w;
}

template <typename T, int RT, bool VEC>
__global__ __launch_bounds__(256) void general_kernel(const AttnParams p, const GenArgs g) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int D = g.head_dim, QS = g.qst;
  float* q_s = smem;                            // [RT][QS]
  float* p_s = q_s + RT * QS;                   // [waves][64 keys][RT]
  float* slab = p_s + kGenWaves * kGenKeys * RT;  // [RT][QS]
  float* ml_s = slab + RT * QS;                 // [waves][RT][2]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const GenWork wk = gen_work(p, g, blockIdx.x);
  const int b = wk.b, h = wk.h;
  int qlen;
  int64_t qoff;
  seq_queries(p, b, qlen, qoff);
  if (p.cu && wk.h == 0 && wk.tile == 0 && wk.split == 0 && tid == 0) {
    const int s0 = p.cu[b], s1 = p.cu[b + 1];
    if (s1 > p.total_tokens || s0 > s1 || s0 < 0) atomicOr(&g_gen_status, kStatusStreamOverrun);
  }
  const int R = qlen * p.n_rep;
  const int r0 = wk.tile * RT;
  // rows past the last tile (a packed sequence longer than the call's max_query_len):
  // zeros, and the status word says so
  if (wk.tile == g.tiles - 1 && wk.split == 0 && R > r0 + RT) {
    if (tid == 0) atomicOr(&g_gen_status, kStatusQueryTooLong);
    for (int64_t idx = tid; idx < (int64_t)(R - r0 - RT) * D; idx += blockDim.x) {
      const int r = r0 + RT + (int)(idx / D), d = (int)(idx % D);
      const int j = r / p.n_rep, hq = h * p.n_rep + (r - j * p.n_rep);
      T* o = (T*)p.out + (int64_t)b * p.o_sb + (qoff + j) * p.o_st + (int64_t)hq * p.o_sh + d;
      *o = (T)0.f;
    }
  }
  if (qlen <= 0 || r0 >= R) return;
  const int ctx = kv_len(p, b);
  const int kvt = gen_kv_tokens(p, ctx);

  // query rows of the tile, fp32, pre-scaled; absent rows and the pad are zero
  for (int idx = tid; idx < RT * QS; idx += blockDim.x) {
    const int rr = idx / QS, d = idx - rr * QS;
    const int r = r0 + rr;
    float v = 0.f;
    if (r < R && d < D) {
      const int j = r / p.n_rep, hq = h * p.n_rep + (r - j * p.n_rep);
      v = to_f32(((const T*)p.q)[(int64_t)b * p.q_sb + (qoff + j) * p.q_st + (int64_t)hq * p.q_sh + d]) *
          p.scale_log2;
    }
    q_s[idx] = v;
  }
  // per-row key limits (uniform): causal end clipped to the reachable keys; 0 for absent rows
  int lim[RT];
  int kmax = 0;
#pragma unroll
  for (int rr = 0; rr < RT; ++rr) {
    const int r = r0 + rr;
    const int j = r / p.n_rep;
    int l = r < R ? ctx - qlen + j + 1 : 0;
    l = l < kvt ? l : kvt;
    lim[rr] = l < 0 ? 0 : l;
    kmax = lim[rr] > kmax ? lim[rr] : kmax;
  }
  const int nblk = (kmax + kGenKeys - 1) / kGenKeys;
  const int per = (nblk + g.ksplit - 1) / g.ksplit;
  const int blk0 = wk.split * per;
  const int blk1 = min(nblk, blk0 + per);
  __syncthreads();

  const int32_t* table = p.bt + (int64_t)b * p.bt_stride;
  const T* kc = (const T*)p.kc;
  const T* vc = (const T*)p.vc;
  const T* zero = (const T*)g_gen_zero;
  const int64_t hoff = (int64_t)h * p.c_sh;
  float* my_p = p_s + wave * kGenKeys * RT;

  float m[RT], l[RT];
  float acc[RT][4];
#pragma unroll
  for (int rr = 0; rr < RT; ++rr) {
    m[rr] = kNegBig;
    l[rr] = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[rr][c] = 0.f;
  }
  constexpr int CH = 16 / (int)sizeof(T);

  for (int kb = blk0 + wave; kb < blk1; kb += kGenWaves) {
    const int key = kb * kGenKeys + lane;
    bool ok = key < kmax;
    int64_t roff = 0;
    if (ok) {
      const int bi = key / p.block_size;
      const int phys = table[bi];
      ok = phys >= 0 && phys < p.num_blocks;
      roff = (int64_t)phys * p.c_sb + (int64_t)(key - bi * p.block_size) * p.c_so + hoff;
    }
    const T* krow = ok ? kc + roff : zero;
    const T* vrow = ok ? vc + roff : zero;
    float s[RT];
#pragma unroll
    for (int rr = 0; rr < RT; ++rr) s[rr] = 0.f;
    if constexpr (VEC) {
      for (int d0 = 0; d0 < D; d0 += CH) {
        float kf[CH];
        widen16<T>(load16(krow + d0), kf);
#pragma unroll
        for (int rr = 0; rr < RT; ++rr) {
          const float* qr = q_s + rr * QS + d0;
#pragma unroll
          for (int e = 0; e < CH; ++e) s[rr] = fmaf(qr[e], kf[e], s[rr]);
        }
      }
    } else {
      for (int d = 0; d < D; ++d) {
        const float kf = to_f32(krow[d]);
#pragma unroll
        for (int rr = 0; rr < RT; ++rr) s[rr] = fmaf(q_s[rr * QS + d], kf, s[rr]);
      }
    }
    const float ninf = -__builtin_inff();
#pragma unroll
    for (int rr = 0; rr < RT; ++rr) {
      const float sv = (ok && key < lim[rr]) ? s[rr] : ninf;
      const float mnew = fmaxf(m[rr], wave_max(sv));
      const float alpha = fast_exp2(m[rr] - mnew);
      const float pv = fast_exp2(sv - mnew);
      l[rr] = l[rr] * alpha + pv;
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[rr][c] *= alpha;
      m[rr] = mnew;
      my_p[lane * RT + rr] = pv;
    }
    // the wave's P slice is read back by every lane of the wave
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int nk = min(kGenKeys, kmax - kb * kGenKeys);
    const uint64_t vaddr = (uint64_t)vrow;
#pragma unroll 4
    for (int k = 0; k < nk; ++k) {
      const uint64_t va = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(vaddr >> 32), k) << 32) |
                          (uint32_t)__builtin_amdgcn_readlane((int)vaddr, k);
      const T* vr = (const T*)va;
      float vf[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d = lane + 64 * c;
        vf[c] = 64 * c < D ? to_f32(vr[d < D ? d : D - 1]) : 0.f;
      }
#pragma unroll
      for (int rr = 0; rr < RT; ++rr) {
        const float pk = my_p[k * RT + rr];
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[rr][c] = fmaf(pk, vf[c], acc[rr][c]);
      }
    }
    // the slice is rewritten by the next block only after every lane has read it
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // merge the waves in wave order
#pragma unroll
  for (int rr = 0; rr < RT; ++rr) {
    l[rr] = wave_sum(l[rr]);
    if (lane == 0) {
      ml_s[(wave * RT + rr) * 2] = m[rr];
      ml_s[(wave * RT + rr) * 2 + 1] = l[rr];
    }
  }
  __syncthreads();
  float M[RT], L[RT], f[RT];
#pragma unroll
  for (int rr = 0; rr < RT; ++rr) {
    float mx = kNegBig;
    for (int w = 0; w < kGenWaves; ++w) mx = fmaxf(mx, ml_s[(w * RT + rr) * 2]);
    float ls = 0.f;
    for (int w = 0; w < kGenWaves; ++w) ls += ml_s[(w * RT + rr) * 2 + 1] * fast_exp2(ml_s[(w * RT + rr) * 2] - mx);
    M[rr] = mx;
    L[rr] = ls;
    f[rr] = fast_exp2(m[rr] - mx);
  }
  for (int w = 0; w < kGenWaves; ++w) {
    if (wave == w) {
#pragma unroll
      for (int rr = 0; rr < RT; ++rr)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int d = lane + 64 * c;
          if (d < D) {
            const float v = acc[rr][c] * f[rr];
            slab[rr * QS + d] = w == 0 ? v : slab[rr * QS + d] + v;
          }
        }
    }
    __syncthreads();
  }
  const int rows = min(RT, R - r0);
  if (g.ksplit == 1) {
    for (int idx = tid; idx < rows * D; idx += blockDim.x) {
      const int rr = idx / D, d = idx - rr * D;
      const int r = r0 + rr;
      const int j = r / p.n_rep, hq = h * p.n_rep + (r - j * p.n_rep);
      float lt = 0.f;
#pragma unroll
      for (int x = 0; x < RT; ++x) lt = x == rr ? L[x] : lt;
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      T* o = (T*)p.out + (int64_t)b * p.o_sb + (qoff + j) * p.o_st + (int64_t)hq * p.o_sh + d;
      *o = (T)(slab[rr * QS + d] * inv);
    }
  } else {
    const int64_t base = (wk.unit * g.ksplit + wk.split) * RT;
    for (int idx = tid; idx < rows * D; idx += blockDim.x) {
      const int rr = idx / D, d = idx - rr * D;
      g.part_o[(base + rr) * D + d] = slab[rr * QS + d];
    }
    if (tid < rows) {
      float mt = 0.f, lt = 0.f;
#pragma unroll
      for (int x = 0; x < RT; ++x) {
        mt = x == tid ? M[x] : mt;
        lt = x == tid ? L[x] : lt;
      }
      g.part_ml[(base + tid) * 2] = mt;
      g.part_ml[(base + tid) * 2 + 1] = lt;
    }
  }
}

// Combines the key splits of one (sequence, KV head, row tile) in split order.
template <typename T, int RT>
__global__ __launch_bounds__(256) void general_merge_kernel(const AttnParams p, const GenArgs g) {
  const int D = g.head_dim;
  const GenWork wk = gen_work(p, g, (int64_t)blockIdx.x * g.ksplit);
  int qlen;
  int64_t qoff;
  seq_queries(p, wk.b, qlen, qoff);
  const int R = qlen * p.n_rep;
  const int r0 = wk.tile * RT;
  if (qlen <= 0 || r0 >= R) return;
  const int rows = min(RT, R - r0);
  const int64_t base = wk.unit * g.ksplit * RT;
  for (int idx = threadIdx.x; idx < rows * D; idx += blockDim.x) {
    const int rr = idx / D, d = idx - rr * D;
    float mx = kNegBig;
    for (int s = 0; s < g.ksplit; ++s) mx = fmaxf(mx, g.part_ml[(base + (int64_t)s * RT + rr) * 2]);
    float ls = 0.f, o = 0.f;
    for (int s = 0; s < g.ksplit; ++s) {
      const int64_t i = base + (int64_t)s * RT + rr;
      const float w = fast_exp2(g.part_ml[i * 2] - mx);
      ls += g.part_ml[i * 2 + 1] * w;
      o += g.part_o[i * D + d] * w;
    }
    const int r = r0 + rr;
    const int j = r / p.n_rep, hq = wk.h * p.n_rep + (r - j * p.n_rep);
    T* out = (T*)p.out + (int64_t)wk.b * p.o_sb + (qoff + j) * p.o_st + (int64_t)hq * p.o_sh + d;
    *out = (T)(ls > 0.f ? o / ls : 0.f);
  }
}

// Launch geometry of a general call.
struct GenPlan {
  int rt, tiles, ksplit;
  int64_t units;
  int64_t ws_bytes;
};

GenPlan gen_plan(int64_t batch, int n_q, int n_kv, int head_dim, int max_query_len, int64_t max_keys) {
  GenPlan pl;
  const int n_rep = n_q / n_kv;
  const int64_t rows = (int64_t)(max_query_len < 1 ? 1 : max_query_len) * n_rep;
  pl.rt = rows <= 1 ? 1 : (rows <= 4 ? 4 : 16);
  pl.tiles = (int)((rows + pl.rt - 1) / pl.rt);
  pl.units = batch * n_kv * (int64_t)pl.tiles;
  // key splits fill about two workgroups per CU when the (sequence, head, tile) units
  // alone do not; each split keeps at least one 64-key block per wave
  const int64_t target = 2 * (int64_t)ss_host::device_cu_count();
  int64_t ks = pl.units >= target ? 1 : target / (pl.units > 0 ? pl.units : 1);
  const int64_t by_keys = (max_keys + kGenKeys * kGenWaves - 1) / (kGenKeys * kGenWaves);
  ks = ks < by_keys ? ks : by_keys;
  ks = ks < kGenMaxSplits ? ks : kGenMaxSplits;
  pl.ksplit = (int)(ks < 1 ? 1 : ks);
  pl.ws_bytes = pl.ksplit > 1 ? pl.units * pl.ksplit * pl.rt * (int64_t)(head_dim + 2) * 4 : 0;
  return pl;
}

template <typename T, int RT, bool VEC>
int launch_general_typed(const AttnParams& p, const GenArgs& g, int64_t units, hipStream_t stream) {
  const size_t lds = (size_t)(2 * RT * g.qst + kGenWaves * kGenKeys * RT + kGenWaves * RT * 2) * sizeof(float);
  hipLaunchKernelGGL((general_kernel<T, RT, VEC>), dim3((unsigned)(units * g.ksplit)), dim3(256), lds, stream, p,
                     g);
  int st = ss_host::launch_status("paged attention (general)");
  if (st != SS_OK || g.ksplit == 1) return st;
  hipLaunchKernelGGL((general_merge_kernel<T, RT>), dim3((unsigned)units), dim3(256), 0, stream, p, g);
  return ss_host::launch_status("paged attention (general) merge");
}

template <typename T, int RT>
int launch_general_rt(const AttnParams& p, const GenArgs& g, int64_t units, bool vec, hipStream_t stream) {
  return vec ? launch_general_typed<T, RT, true>(p, g, units, stream)
             : launch_general_typed<T, RT, false>(p, g, units, stream);
}

template <typename T>
int launch_general_t(const AttnParams& p, const GenArgs& g, int rt, int64_t units, bool vec, hipStream_t stream) {
  if (rt == 1) return launch_general_rt<T, 1>(p, g, units, vec, stream);
  if (rt == 4) return launch_general_rt<T, 4>(p, g, units, vec, stream);
  return launch_general_rt<T, 16>(p, g, units, vec, stream);
}

}  // namespace

// Workspace of a general call (the key-split partials; 0 when there is one split).
// Bounded independently of the batch: the splits fill at most two workgroups per CU.
int64_t general_workspace_bytes(int64_t batch, int n_q, int n_kv, int head_dim, int max_query_len,
                                int64_t max_keys) {
  return (gen_plan(batch, n_q, n_kv, head_dim, max_query_len, max_keys).ws_bytes + 255) & ~(int64_t)255;
}

// Upper bound of general_workspace_bytes over every batch and table width.
int64_t general_workspace_bound(int n_q, int n_kv, int head_dim, int max_query_len) {
  (void)n_q;
  (void)n_kv;
  (void)max_query_len;
  const int64_t target = 2 * (int64_t)ss_host::device_cu_count();
  return ((target * 16 * (int64_t)(head_dim + 2) * 4) + 255) & ~(int64_t)255;
}

// vec: 16-byte row loads allowed (rows and strides of the cache planes 16-byte aligned).
int launch_general(const AttnParams& p, int dtype, int head_dim, int max_query_len, bool vec, void* ws,
                   int64_t ws_bytes, hipStream_t stream) {
  const int64_t max_keys = (int64_t)p.max_blocks * p.block_size;
  const GenPlan pl = gen_plan(p.batch, p.n_q, p.n_kv, head_dim, max_query_len, max_keys);
  if (pl.ws_bytes > 0 && (!ws || ws_bytes < pl.ws_bytes)) {
    ss_host::set_error("paged attention (general): workspace of %lld bytes, needs %lld", (long long)ws_bytes,
                       (long long)pl.ws_bytes);
    return SS_ERR_WORKSPACE;
  }
  if ((int64_t)pl.units * pl.ksplit > 0x7fffffffll) {
    ss_host::set_error("paged attention (general): grid of %lld workgroups too large",
                       (long long)(pl.units * pl.ksplit));
    return SS_ERR_UNSUPPORTED;
  }
  GenArgs g;
  g.head_dim = head_dim;
  g.qst = (head_dim + 3) & ~3;
  g.tiles = pl.tiles;
  g.ksplit = pl.ksplit;
  g.part_ml = (float*)ws;
  g.part_o = pl.ksplit > 1 ? (float*)ws + pl.units * pl.ksplit * pl.rt * 2 : nullptr;
  if (dtype == SS_DTYPE_F32) return launch_general_t<float>(p, g, pl.rt, pl.units, vec, stream);
  if (dtype == SS_DTYPE_BF16) return launch_general_t<bf16_t>(p, g, pl.rt, pl.units, vec, stream);
  return launch_general_t<f16_t>(p, g, pl.rt, pl.units, vec, stream);
}

// Status word of the general kernels: queue its atomic take on `stream`, then (after
// the stream has been synchronised) read the value taken.
int general_status_take(int clear, hipStream_t stream) {
  hipLaunchKernelGGL(gen_status_take_kernel, dim3(1), dim3(1), 0, stream, clear);
  return hipGetLastError() == hipSuccess ? SS_OK : SS_ERR_LAUNCH;
}

int general_status_value(int* v) {
  return hipMemcpyFromSymbol(v, HIP_SYMBOL(g_gen_status_seen), sizeof(int), 0, hipMemcpyDeviceToHost) == hipSuccess
             ? SS_OK
             : SS_ERR_LAUNCH;
}

}  // namespace ss
