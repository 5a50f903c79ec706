// Split-K paged-attention decode for gfx950.
//
// Math (slipstream/models/layers/attention.py:64-88 via
// slipstream/kernels/attention_ref.py:68-89, edge rules of
// slipstream/kernels/triton_paged.py:133-206): for query row r = (token j, head
// i of the GQA group of KV head h) of sequence b,
//   out = softmax(scale * q . K^T + causal) . V
// over the first ctx(b) tokens gathered through block_tables[b].
//
// Work partition ("stream-K"): the decode sequences' KV is cut into pairs of
// 16-token tiles (32 keys). All pairs of all sequences form one list, in
// sequence order; workgroup w takes the contiguous range
// [w*chunk, (w+1)*chunk). A workgroup has one wavefront per KV head of its head
// group, so its waves stream the same pages of the same blocks (contiguous
// [block, offset, head, d] memory). A sequence finished inside one range is
// written directly; a sequence cut by a range boundary leaves an unnormalised
// partial (max, sum, acc) per range, and the merge kernel combines them. Every
// workgroup gets the same number of pairs, whatever the length distribution.
//
// Per wavefront and pair:
//   S^T = K Q^T   : 2 tiles x D/32 MFMA 16x16x32 (A = K rows straight from
//                   HBM in MFMA layout, B = Q^T held in registers)
//   online softmax in fp32 (exp2 domain), max across the 4 lane rows with
//                   v_permlane{16,32}_swap
//   O^T += V^T P^T: D/8/16 x 8 MFMA; V is loaded as whole 256-byte rows (each
//                   lane 8 tokens x 8 consecutive d) and transposed inside the
//                   lane with v_perm_b32, because MFMA row m of product i stands
//                   for d = 8*m + i. P^T comes straight out of the S^T
//                   accumulator layout. No LDS is used.
#include "attention_common.h"
#include "prefill_tile.h"

namespace ss {
namespace {

// Target of every load for an absent key (past the context, or in a block whose
// table entry is negative or out of range). Never written, so it stays zero.
__device__ __attribute__((aligned(16))) uint32_t g_zero_row[128];

// Device status word of this GPU (kStatus* bits), read and cleared by
// ss_attention_status. Kernels only OR bits into it.
__device__ int g_status;
// The word as status_take_kernel last read it.
__device__ int g_status_seen;

// One thread: take the status word (exchange with 0 when clearing, else read it
// through an atomic that changes nothing) and leave it where the host copies it from.
__global__ void status_take_kernel(int clear) {
  g_status_seen = clear ? atomicExch(&g_status, 0) : atomicOr(&g_status, 0);
}

__device__ __forceinline__ int block_sum(int v, int* sh) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) sh[wave] = v;
  __syncthreads();
  int t = 0;
  for (int i = 0; i < nw; ++i) t += sh[i];
  return t;
}

__device__ __forceinline__ int block_incl_scan(int v, int* sh, int& total) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(v, o);
    if (lane >= o) v += u;
  }
  __syncthreads();
  if (lane == 63) sh[wave] = v;
  __syncthreads();
  int pre = 0;
  total = 0;
  for (int i = 0; i < nw; ++i) {
    const int s = sh[i];
    if (i < wave) pre += s;
    total += s;
  }
  return v + pre;
}

// Pairs of 16-token tiles the decode kernel owns for sequence b (0 for
// sequences left to the prefill kernel or with nothing to attend to).
__device__ __forceinline__ int decode_pairs(const AttnParams& p, int b) {
  int qlen;
  int64_t qoff;
  seq_queries(p, b, qlen, qoff);
  if (!is_decode_seq(p, qlen)) return 0;
  const int kvt = seq_kv_tokens(p, kv_len(p, b));
  return (kvt + kPairTokens - 1) / kPairTokens;
}

template <typename T, int D>
struct DecodeTile {
  static constexpr int NCH = D / 8;             // 16-byte chunks in a head row
  static constexpr int MT = (NCH + 15) / 16;    // PV product sets (16 chunks each)
  static constexpr int KS = D / 32;             // QK k-steps
  u32x4 k[2][KS];   // A operands of S^T: row = token (lane & 15), k = d
  u32x4 v[MT][8];   // 8 tokens of lane row g x 8 consecutive d of chunk (lane & 15) + 16*mt
  int valid;        // bit x: tile x of this lane row's V tokens lives in a valid block
};

// The block-table entries a lane needs for pair `pi`: the block of its K token (tile x)
// and of its V tokens (tile x).
struct PairPhys {
  int k[2];
  int v[2];
};

__device__ __forceinline__ PairPhys fetch_pair_phys(const AttnParams& p, const int32_t* table, int pi, int lane) {
  const int n = lane & 15, g = lane >> 4;
  PairPhys ph;
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    int bk = (pi * kPairTokens + 16 * x + n) >> p.bs_shift;
    int bv = (pi * kPairTokens + 16 * x + 4 * g) >> p.bs_shift;
    ph.k[x] = table[bk < p.max_blocks ? bk : p.max_blocks - 1];
    ph.v[x] = table[bv < p.max_blocks ? bv : p.max_blocks - 1];
  }
  return ph;
}

// Issue the K/V loads of pair `pi` given its table entries. Every load is
// unconditional: absent keys read the zero row instead.
template <typename T, int D>
__device__ __forceinline__ void load_pair_phys(const AttnParams& p, const PairPhys& ph, int kvt, int pi, int h,
                                               int lane, DecodeTile<T, D>& t) {
  typedef DecodeTile<T, D> Tile;
  const char* kc = (const char*)p.kc;
  const char* vc = (const char*)p.vc;
  const char* zero = (const char*)g_zero_row;
  const int n = lane & 15, g = lane >> 4;
  const int bmask = p.block_size - 1;
  const int64_t hoff = (int64_t)h * p.c_sh;
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    // K: this lane's token is n of tile x
    const int tk = pi * kPairTokens + 16 * x + n;
    const int phys = ph.k[x];
    const bool ok = tk < kvt && phys >= 0 && phys < p.num_blocks;
    const char* krow =
        ok ? kc + ((int64_t)phys * p.c_sb + (int64_t)(tk & bmask) * p.c_so + hoff) * (int64_t)sizeof(T)
           : zero;
#pragma unroll
    for (int s = 0; s < Tile::KS; ++s) t.k[x][s] = load16(krow + (32 * s + 8 * g) * (int)sizeof(T));
  }
  t.valid = 0;
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    // V: tokens 4g..4g+3 of tile x share one block (block_size >= 4)
    const int t0 = pi * kPairTokens + 16 * x + 4 * g;
    const int phys = ph.v[x];
    const bool okb = phys >= 0 && phys < p.num_blocks;
    if (okb) t.valid |= 1 << x;
    const int64_t base = ((int64_t)phys * p.c_sb + hoff) * (int64_t)sizeof(T);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int tv = t0 + e;
      const char* vrow = (okb && tv < kvt) ? vc + base + (int64_t)(tv & bmask) * p.c_so * (int64_t)sizeof(T)
                                           : zero;
#pragma unroll
      for (int mt = 0; mt < Tile::MT; ++mt) {
        const int cc = n + 16 * mt;
        const int ccl = cc < Tile::NCH ? cc : 0;
        t.v[mt][4 * x + e] = load16(vrow + 8 * ccl * (int)sizeof(T));
      }
    }
  }
}

// Issue the loads of pair `pi` of the sequence whose table is `table`.
template <typename T, int D>
__device__ __forceinline__ void load_pair(const AttnParams& p, const int32_t* table, int kvt, int pi,
                                          int h, int lane, DecodeTile<T, D>& t) {
  load_pair_phys<T, D>(p, fetch_pair_phys(p, table, pi, lane), kvt, pi, h, lane, t);
}

template <typename T, int D>
struct RowState {
  static constexpr int NACC = DecodeTile<T, D>::MT * 8;
  f32x4 acc[NACC];  // acc[mt*8+i][e] = O[row][128*mt + 32*g + 8*e + i]
  float m;          // running max (log2 domain), uniform over the lanes of a row
  float l;          // this lane's partial sum of exp2(s - m)
};

// Shared-prefix cascade: fold the p.px_n normalised prefix parts of query row
// `row` (b * n_q + hq) into a running state -- max m and sum l (log2 domain), the
// unnormalised output o[2c], o[2c + 1] of the 8 consecutive d at d0 + 8c -- as
// parts of weight 2^(lse_s - M) against the state's 2^(m - M): the softmax over a
// union of disjoint key sets is the lse-weighted mix of the parts' softmaxes.
// The loads of SB parts are issued before any is used. Every part holds at least
// one key (finite lse), so M is finite after the first batch.
template <typename T, int D, int NC, int SB>
__device__ __forceinline__ void fold_prefix(const AttnParams& p, int64_t row, int d0, float& m, float& l,
                                            f32x4 (&o)[2 * NC]) {
  const int64_t rows = (int64_t)p.batch * p.n_q;
  const T* part = (const T*)p.px_part;
  for (int s0 = 0; s0 < p.px_n; s0 += SB) {
    float lv[SB];
    u32x4 v[SB][NC];
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      const int64_t i = (int64_t)min(s0 + j, p.px_n - 1) * rows + row;
      lv[j] = p.px_lse[i];
#pragma unroll
      for (int c = 0; c < NC; ++c) v[j][c] = load16(part + i * D + d0 + 8 * c);
    }
    float mx = m;
#pragma unroll
    for (int j = 0; j < SB; ++j) mx = s0 + j < p.px_n ? fmaxf(mx, lv[j]) : mx;
    const float keep = fast_exp2(m - mx);
    l *= keep;
#pragma unroll
    for (int c = 0; c < 2 * NC; ++c) o[c] *= keep;
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      const float w = s0 + j < p.px_n ? fast_exp2(lv[j] - mx) : 0.f;
      l += w;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        o[2 * c] += w * f32x4{Elem<T>::lo(v[j][c][0]), Elem<T>::hi(v[j][c][0]), Elem<T>::lo(v[j][c][1]),
                              Elem<T>::hi(v[j][c][1])};
        o[2 * c + 1] += w * f32x4{Elem<T>::lo(v[j][c][2]), Elem<T>::hi(v[j][c][2]), Elem<T>::lo(v[j][c][3]),
                                  Elem<T>::hi(v[j][c][3])};
      }
    }
    m = mx;
  }
}

// lim_min: the smallest per-row key limit of this wave's rows (wave-uniform). A pair
// whose tiles are both valid and end at or before lim_min needs no masking.
template <typename T, int D>
__device__ __forceinline__ void compute_pair(const AttnParams& p, const DecodeTile<T, D>& t,
                                             const u32x4 (&qop)[D / 32], int pi, int lim_eff, int lim_min,
                                             int lane, RowState<T, D>& st) {
  typedef DecodeTile<T, D> Tile;
  const int g = lane >> 4;
  f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < Tile::KS; ++s) {
    s0 = Elem<T>::mfma(t.k[0][s], qop[s], s0);
    s1 = Elem<T>::mfma(t.k[1][s], qop[s], s1);
  }
  // s0[e] = S[token pi*32 + 4g + e][row], s1[e] = S[token pi*32 + 16 + 4g + e][row]
  float sv[8];
  const bool full = (pi + 1) * kPairTokens <= lim_min && __all(t.valid == 3);
  if (full) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sv[e] = s0[e] * p.scale_log2;
      sv[4 + e] = s1[e] * p.scale_log2;
    }
  } else {
    const int tb = pi * kPairTokens + 4 * g;
    const float ninf = -__builtin_inff();
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sv[e] = ((t.valid & 1) && tb + e < lim_eff) ? s0[e] * p.scale_log2 : ninf;
      sv[4 + e] = ((t.valid & 2) && tb + 16 + e < lim_eff) ? s1[e] * p.scale_log2 : ninf;
    }
  }
  float mx = sv[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) mx = fmaxf(mx, sv[e]);
  mx = max_across_rows(mx);
  const float mnew = fmaxf(st.m, mx);
  // Rescale only when some row's running max grew (exact: alpha is 1 otherwise); after
  // the first few pairs of a sequence the max rarely moves.
  if (__any(mnew > st.m)) {
    const float alpha = fast_exp2(st.m - mnew);
    st.l *= alpha;
#pragma unroll
    for (int a = 0; a < RowState<T, D>::NACC; ++a) st.acc[a] *= alpha;
  }
  st.m = mnew;
  float pv[8];
  float ps = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    pv[e] = fast_exp2(sv[e] - mnew);
    ps += pv[e];
  }
  st.l += ps;
  const u32x4 pop = {Elem<T>::pack2(pv[0], pv[1]), Elem<T>::pack2(pv[2], pv[3]),
                     Elem<T>::pack2(pv[4], pv[5]), Elem<T>::pack2(pv[6], pv[7])};
#pragma unroll
  for (int mt = 0; mt < Tile::MT; ++mt) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      u32x4 a;
      if (i & 1) {
        a[0] = pick_halves<1, 1>(t.v[mt][0][i >> 1], t.v[mt][1][i >> 1]);
        a[1] = pick_halves<1, 1>(t.v[mt][2][i >> 1], t.v[mt][3][i >> 1]);
        a[2] = pick_halves<1, 1>(t.v[mt][4][i >> 1], t.v[mt][5][i >> 1]);
        a[3] = pick_halves<1, 1>(t.v[mt][6][i >> 1], t.v[mt][7][i >> 1]);
      } else {
        a[0] = pick_halves<0, 0>(t.v[mt][0][i >> 1], t.v[mt][1][i >> 1]);
        a[1] = pick_halves<0, 0>(t.v[mt][2][i >> 1], t.v[mt][3][i >> 1]);
        a[2] = pick_halves<0, 0>(t.v[mt][4][i >> 1], t.v[mt][5][i >> 1]);
        a[3] = pick_halves<0, 0>(t.v[mt][6][i >> 1], t.v[mt][7][i >> 1]);
      }
      st.acc[mt * 8 + i] = Elem<T>::mfma(a, pop, st.acc[mt * 8 + i]);
    }
  }
}

// ---- small decode batches (one launch, no merge)
//
// For a padded decode call with few (sequence, KV head) pairs and short tables, one
// workgroup per (sequence b, KV head h): its eight waves take the same query rows (the
// qlen * n_rep <= 16 rows of the split-K kernel's tile) and an eighth of the sequence's
// 32-key pairs each, with the decode's pair loads and pair math; wave 0 then combines
// the eight (max, sum, output) states through LDS by log-sum-exp weight and writes the
// rows. Every row of the call is written here (a sequence with no key gets zeros, as
// the merge writes them), so no merge kernel follows: for C1-sized calls the split-K
// launch's plan scan and its merge launch are most of the time.
template <typename T, int D>
__global__ __launch_bounds__(512) void decode_small_kernel(const AttnParams p) {
  typedef DecodeTile<T, D> Tile;
  constexpr int NW = 8;
  constexpr int NACC = RowState<T, D>::NACC;
  __shared__ float s_ml[NW][16][2];
  __shared__ f32x4 s_acc[NW - 1][NACC][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int b = blockIdx.x / p.n_kv, h = blockIdx.x - (blockIdx.x / p.n_kv) * p.n_kv;
  int qlen;
  int64_t qoff;
  seq_queries(p, b, qlen, qoff);
  qlen = __builtin_amdgcn_readfirstlane(qlen);
  const int R = qlen * p.n_rep;
  const bool row_ok = n < R;
  const int j = row_ok ? n / p.n_rep : 0;
  const int hq = h * p.n_rep + (row_ok ? n - j * p.n_rep : 0);
  // wave w takes pairs w, w + NW, ...: its first pair's table entries and K/V rows are
  // requested before the sequence's length arrives (through the whole table, every
  // block checked), and the V rows past the length are zeroed once it has (keys past
  // it are masked by the pair math; a zero V row keeps stale values of unused slots
  // out of the product)
  const int32_t* table = p.bt + (int64_t)b * p.bt_stride;
  const int cap = p.max_blocks << p.bs_shift;
  DecodeTile<T, D> ta, tb;
  {
    // the table entries of both first pairs before any K/V load: a table load issued
    // behind K/V loads waits for them (the vector-memory counter retires in order)
    const PairPhys pa = fetch_pair_phys(p, table, wave, lane);
    const PairPhys pb = fetch_pair_phys(p, table, wave + NW, lane);
    load_pair_phys<T, D>(p, pa, cap, wave, h, lane, ta);
    load_pair_phys<T, D>(p, pb, cap, wave + NW, h, lane, tb);
  }
  const int ctx = __builtin_amdgcn_readfirstlane(kv_len(p, b));
  const int kvt = seq_kv_tokens(p, ctx);
  const int lim = row_ok ? ctx - qlen + j + 1 : 0;
  const int lim_eff = lim < kvt ? lim : kvt;
  int lim_min = row_ok ? lim_eff : 0x7fffffff;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) lim_min = min(lim_min, __shfl_xor(lim_min, o));
  lim_min = __builtin_amdgcn_readfirstlane(lim_min);
  u32x4 qop[Tile::KS];
  {
    const T* qrow = (const T*)p.q + (int64_t)b * p.q_sb + (qoff + j) * p.q_st + (int64_t)hq * p.q_sh;
#pragma unroll
    for (int s2 = 0; s2 < Tile::KS; ++s2) {
      const u32x4 z = {0u, 0u, 0u, 0u};
      qop[s2] = row_ok ? load16(qrow + 32 * s2 + 8 * g) : z;
    }
  }
  RowState<T, D> st;
#pragma unroll
  for (int a = 0; a < NACC; ++a) st.acc[a] = f32x4{0.f, 0.f, 0.f, 0.f};
  st.m = kNegBig;
  st.l = 0.f;
  const int npairs = (kvt + kPairTokens - 1) / kPairTokens;
  int pi = wave;
  if (pi < npairs) {
    // the first two pairs were loaded through the whole table: zero their V rows past
    // the length
    auto zero_v_past = [&](DecodeTile<T, D>& t, int pt) {
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool live = pt * kPairTokens + 16 * x + 4 * g + e < kvt;
#pragma unroll
          for (int mt = 0; mt < Tile::MT; ++mt)
            t.v[mt][4 * x + e] = live ? t.v[mt][4 * x + e] : u32x4{0u, 0u, 0u, 0u};
        }
    };
    zero_v_past(ta, pi);
    zero_v_past(tb, pi + NW);
    compute_pair<T, D>(p, ta, qop, pi, lim_eff, lim_min, lane, st);
    pi += NW;
    while (pi < npairs) {  // tb holds pair pi
      load_pair<T, D>(p, table, kvt, pi + NW, h, lane, ta);
      compute_pair<T, D>(p, tb, qop, pi, lim_eff, lim_min, lane, st);
      pi += NW;
      if (pi >= npairs) break;
      load_pair<T, D>(p, table, kvt, pi + NW, h, lane, tb);
      compute_pair<T, D>(p, ta, qop, pi, lim_eff, lim_min, lane, st);
      pi += NW;
    }
  }
  const float lt = sum_across_rows(st.l);
  if (g == 0) {
    s_ml[wave][n][0] = st.m;
    s_ml[wave][n][1] = lt;
  }
  if (wave > 0) {
#pragma unroll
    for (int a = 0; a < NACC; ++a) s_acc[wave - 1][a][lane] = st.acc[a];
  }
  __syncthreads();
  if (wave != 0 || !row_ok) return;
  // log-sum-exp combination of the waves' states (a wave without pairs has max
  // kNegBig and sum 0; if no wave had a key the sum stays 0 and the row is zeros)
  float mx = st.m;
#pragma unroll
  for (int w = 1; w < NW; ++w) mx = fmaxf(mx, s_ml[w][n][0]);
  const float f0 = fast_exp2(st.m - mx);
  float lsum = lt * f0;
#pragma unroll
  for (int a = 0; a < NACC; ++a) st.acc[a] *= f0;
  // One wave's state ahead of the adds: left to itself the compiler sank the adds to
  // the output stores, kept all seven states of 32 floats live beside the lane's own and
  // spilled. The empty asm makes each wave's sums exist before the wave after next is
  // read; the next wave's state is requested before them, so its LDS latency overlaps.
  f32x4 cur[NACC];
#pragma unroll
  for (int a = 0; a < NACC; ++a) cur[a] = s_acc[0][a][lane];
#pragma unroll
  for (int w = 1; w < NW; ++w) {
    f32x4 nxt[NACC];
    if (w + 1 < NW) {
#pragma unroll
      for (int a = 0; a < NACC; ++a) nxt[a] = s_acc[w][a][lane];
    }
    const float f = fast_exp2(s_ml[w][n][0] - mx);
    lsum += f * s_ml[w][n][1];
#pragma unroll
    for (int a = 0; a < NACC; ++a) {
      st.acc[a] += f * cur[a];
      asm volatile("" : "+v"(st.acc[a]));
    }
    if (w + 1 < NW) {
#pragma unroll
      for (int a = 0; a < NACC; ++a) cur[a] = nxt[a];
    }
  }
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  if (p.lse && g == 0) p.lse[lse_index(p, b, qoff, j, hq)] = row_lse(mx, lsum);
  T* orow = (T*)p.out + (int64_t)b * p.o_sb + (qoff + j) * p.o_st + (int64_t)hq * p.o_sh;
#pragma unroll
  for (int mt = 0; mt < Tile::MT; ++mt) {
    const int dbase = 128 * mt + 32 * g;
    if (dbase < D) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f32x4* a = &st.acc[mt * 8];
        const u32x4 o = {Elem<T>::pack2(a[0][e] * inv, a[1][e] * inv), Elem<T>::pack2(a[2][e] * inv, a[3][e] * inv),
                         Elem<T>::pack2(a[4][e] * inv, a[5][e] * inv), Elem<T>::pack2(a[6][e] * inv, a[7][e] * inv)};
        store16(orow + dbase + 8 * e, o);
      }
    }
  }
}

// ---- scalar block-table path (block_size >= 16: a 16-token tile lies in one block)
//
// The tile's physical block is wave-uniform, so its table entry is a scalar load
// (constant address space), fetched one pair ahead on the scalar memory counter --
// waiting for it never waits for the K/V vector loads in flight. Each tile is read
// through a buffer descriptor whose base is the tile's first token in the layer plane
// and whose size covers exactly its valid tokens: loads past the context or from an
// absent block (size 0) return zeros in hardware, and every lane's byte offset is a
// constant of the kernel, so a pair costs no vector address arithmetic.
typedef const __attribute__((address_space(4))) int32_t* ConstTable;

// Cache policy of the K/V page loads (buffer-load aux bits). A page read once per step
// streams best non-temporally: without allocating in the caches it measured ~14 % more
// bandwidth on gfx950 than the default policy. Pages shared by several sequences (a
// common prefix) are read once per sequence, and there the default policy lets the
// re-reads hit the 256 MB MALL; the host picks the policy from the pool's size.
constexpr int kNonTemporal = 2;
constexpr int kDefaultPolicy = 0;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const char* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), (short)0, bytes, 0x00020000);
}

struct ScalarTableCtx {
  const char* kplane;
  const char* vplane;
  ConstTable table;  // this sequence's block-table row
  int64_t blk_bytes;  // one block of one plane
  int tok_bytes;      // one token (all heads) of one plane
  int kvt;            // KV tokens reachable through the table
};

// Physical blocks of the two tiles of pair pj (-1: absent or past the table).
__device__ __forceinline__ void fetch_phys(const AttnParams& p, const ScalarTableCtx& c, int pj, int (&ph)[2]) {
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const int bi = (pj * kPairTokens + 16 * x) >> p.bs_shift;
    const int v = c.table[bi < p.max_blocks ? bi : p.max_blocks - 1];
    ph[x] = (bi < p.max_blocks && v >= 0 && v < p.num_blocks) ? v : -1;
  }
}

template <typename T, int D, int AUX>
__device__ __forceinline__ void load_pair_scalar(const AttnParams& p, const ScalarTableCtx& c, int pi,
                                                 const int (&ph)[2], int voff_k, const int (&voff_v)[4],
                                                 DecodeTile<T, D>& t) {
  typedef DecodeTile<T, D> Tile;
  const int bmask = p.block_size - 1;
  t.valid = 0;
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const int tok = pi * kPairTokens + 16 * x;
    const int bi = tok >> p.bs_shift;
    const int tib = tok & bmask;
    const bool ok = ph[x] >= 0;
    int vt = c.kvt - (bi << p.bs_shift);  // valid tokens of the block
    vt = vt < 0 ? 0 : (vt > p.block_size ? p.block_size : vt);
    const int live = vt > tib ? vt - tib : 0;
    // offset and size through readfirstlane: they are uniform, but where the compiler
    // cannot prove it (a select on a lane mask) it wraps every load of the tile in a
    // waterfall loop over the descriptor
    int64_t off = ok ? (int64_t)ph[x] * c.blk_bytes + (int64_t)tib * c.tok_bytes : 0;
    off = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(off >> 32)) << 32) |
                    (uint32_t)__builtin_amdgcn_readfirstlane((int)off));
    const int bytes = __builtin_amdgcn_readfirstlane(ok ? live * c.tok_bytes : 0);
    if (ok) t.valid |= 1 << x;
    const __amdgpu_buffer_rsrc_t rk = tile_rsrc(c.kplane + off, bytes);
    const __amdgpu_buffer_rsrc_t rv = tile_rsrc(c.vplane + off, bytes);
#pragma unroll
    for (int s = 0; s < Tile::KS; ++s)
      t.k[x][s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, voff_k + 64 * s, 0, AUX));
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int mt = 0; mt < Tile::MT; ++mt)
        t.v[mt][4 * x + e] =
            __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, voff_v[e] + 256 * mt, 0, AUX));
  }
}

// STAB: scalar block-table path (block_size >= 16); otherwise every lane looks up
// its own block (block_size 4 and 8 put several blocks in one 16-token tile). AUX: the
// page-load cache policy of the STAB path.
// The body of decode_kernel as workgroup bid. CASCADE: the shared-prefix cascade runs
// it in the eight-wave workgroups after its prefix pass, each half of the waves
// (0-3, 4-7) on a range of its own (ranges 2 bid and 2 bid + 1): both halves take
// part in the plan's block reductions, then waves past hpw in each half leave.
template <typename T, int D, bool STAB, int AUX, bool CASCADE>
__device__ __forceinline__ void decode_body(const AttnParams& p, const unsigned bid) {
  typedef DecodeTile<T, D> Tile;
  __shared__ int s_red[16];
  __shared__ int s_b0[2], s_c0[2];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave_wg = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = CASCADE ? wave_wg >> 2 : 0;
  const int wave = CASCADE ? wave_wg & 3 : wave_wg;  // the wave's KV head within its group
  const unsigned vb = CASCADE ? 2 * bid + half : bid;  // (range, head group) of the wave
  const int n = lane & 15, g = lane >> 4;
  const int hg = vb % p.n_hgroups;  // unsigned: no sign fix-ups in the division
  const int wr = vb / p.n_hgroups;
  const int h = hg * p.hpw + wave;
  int* rec = p.ws_rec + (int64_t)vb * 8;
  const bool rec_writer = CASCADE ? (tid & 255) == 0 : tid == 0;

  // ---- plan: total pairs, this range, and the sequence holding its first pair
  // pair count of this thread's first sequence, kept for the scan's first pass (one
  // memory round trip less before the stream starts when the batch fits one pass)
  const int v_first = tid < p.batch ? decode_pairs(p, tid) : 0;
  int local = v_first;
  for (int b = tid + blockDim.x; b < p.batch; b += blockDim.x) local += decode_pairs(p, b);
  // the plan's values are wave-uniform (block reductions); readfirstlane tells the
  // compiler so, which keeps the pair loop's scalars and buffer descriptors in SGPRs
  const int total = __builtin_amdgcn_readfirstlane(block_sum(local, s_red));
  const int chunk = (total + p.n_ranges - 1) / p.n_ranges;
  const int s_w = wr * chunk;
  const int e_w = min(s_w + chunk, total);
  if constexpr (!CASCADE) {
    if (s_w >= e_w) {
      if (tid == 0) {
        rec[0] = -1;
        rec[5] = -1;
      }
      return;
    }
    if (tid == 0) s_b0[0] = -1;
    int run = 0;
    for (int base = 0; base < p.batch; base += blockDim.x) {
      const int b = base + tid;
      const int v = base == 0 ? v_first : (b < p.batch ? decode_pairs(p, b) : 0);
      int tot;
      const int incl = block_incl_scan(v, s_red, tot);
      const int cb = run + incl - v;
      if (v > 0 && cb <= s_w && s_w < cb + v) {
        s_b0[0] = b;
        s_c0[0] = cb;
      }
      run += tot;
      __syncthreads();
      if (s_b0[0] >= 0) break;
    }
  } else {
    // the first pair of both halves' ranges; a half with an empty range is marked
    // found (-2) from the start, so the scan ends when both are known
    const int sw2[2] = {(int)((2 * bid) / p.n_hgroups) * chunk, (int)((2 * bid + 1) / p.n_hgroups) * chunk};
    if (tid < 2) s_b0[tid] = sw2[tid] < min(sw2[tid] + chunk, total) ? -1 : -2;
    int run = 0;
    for (int base = 0; base < p.batch; base += blockDim.x) {
      const int b = base + tid;
      const int v = base == 0 ? v_first : (b < p.batch ? decode_pairs(p, b) : 0);
      int tot;
      const int incl = block_incl_scan(v, s_red, tot);
      const int cb = run + incl - v;
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        if (v > 0 && cb <= sw2[x] && sw2[x] < cb + v) {
          s_b0[x] = b;
          s_c0[x] = cb;
        }
      }
      run += tot;
      __syncthreads();
      if (s_b0[0] != -1 && s_b0[1] != -1) break;
    }
    // no barrier follows: a half with nothing to do, and waves past hpw, leave here
    if (s_w >= e_w) {
      if (rec_writer) {
        rec[0] = -1;
        rec[5] = -1;
      }
      return;
    }
    if (wave >= p.hpw) return;
  }
  int b = __builtin_amdgcn_readfirstlane(s_b0[half]), c = __builtin_amdgcn_readfirstlane(s_c0[half]), pos = s_w;
  // lane byte offsets of the scalar-table path: constant for the whole kernel
  const int tok_bytes = (int)(p.c_so * (int64_t)sizeof(T));
  const int head_bytes = (int)(p.c_sh * (int64_t)sizeof(T));
  const int voff_k = n * tok_bytes + h * head_bytes + 16 * g;
  int voff_v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) voff_v[e] = (4 * g + e) * tok_bytes + h * head_bytes + 16 * (n < Tile::NCH ? n : 0);
  int rec_b = -1, rec_cb = 0, rec_cb1 = 0, rec_slot = 0;
  int rec_c0 = -1, rec_c1 = -1;  // sequences [rec_c0, rec_c1) finished here, cascade only
  // Write a finished segment: the output rows when it covers the whole sequence,
  // else an unnormalised partial (max, sum, acc) for the merge kernel.
  auto finish = [&](int b, int c, int64_t qoff, int j, int hq, bool row_ok, int seg0, int seg1, int nbp,
                    const RowState<T, D>& st) {
  const float lt = sum_across_rows(st.l);
      const bool complete = seg0 == 0 && seg1 == nbp;
      if (complete && p.px_n == 0) {
        if (row_ok) {
          const float inv = lt > 0.f ? 1.f / lt : 0.f;
          if (p.lse && g == 0) p.lse[lse_index(p, b, qoff, j, hq)] = row_lse(st.m, lt);
          T* orow = (T*)p.out + (int64_t)b * p.o_sb + (qoff + j) * p.o_st + (int64_t)hq * p.o_sh;
#pragma unroll
          for (int mt = 0; mt < Tile::MT; ++mt) {
            const int dbase = 128 * mt + 32 * g;
            if (dbase < D) {
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const f32x4* a = &st.acc[mt * 8];
                const u32x4 o = {Elem<T>::pack2(a[0][e] * inv, a[1][e] * inv),
                                 Elem<T>::pack2(a[2][e] * inv, a[3][e] * inv),
                                 Elem<T>::pack2(a[4][e] * inv, a[5][e] * inv),
                                 Elem<T>::pack2(a[6][e] * inv, a[7][e] * inv)};
                store16(orow + dbase + 8 * e, o);
              }
            }
          }
        }
      } else {
        // a partial: this range's piece of a split sequence, or (shared-prefix cascade)
        // a sequence finished here, which the merge completes with the prefix parts
        const int slot = c > s_w ? 1 : 0;
        const int64_t pidx = complete ? lse_index(p, b, qoff, j, hq)
                                      : (((int64_t)vb * 2 + slot) * p.hpw + wave) * p.rmax + n;
        if (row_ok) {
          float* po = (complete ? p.px_seq_o : p.ws_o) + pidx * D;
#pragma unroll
          for (int mt = 0; mt < Tile::MT; ++mt) {
            const int dbase = 128 * mt + 32 * g;
            if (dbase < D) {
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const f32x4* a = &st.acc[mt * 8];
                const f32x4 lo = {a[0][e], a[1][e], a[2][e], a[3][e]};
                const f32x4 hi = {a[4][e], a[5][e], a[6][e], a[7][e]};
                *reinterpret_cast<f32x4*>(po + dbase + 8 * e) = lo;
                *reinterpret_cast<f32x4*>(po + dbase + 8 * e + 4) = hi;
              }
            }
          }
          if (g == 0) {
            float* pml = (complete ? p.px_seq_ml : p.ws_ml) + pidx * 2;
            pml[0] = st.m;
            pml[1] = lt;
          }
        }
        if (complete) {
          rec_c0 = rec_c0 < 0 ? b : rec_c0;
          rec_c1 = b + 1;
        } else if (c >= s_w) {
          rec_b = b;
          rec_cb = c;
          rec_cb1 = c + nbp;
          rec_slot = slot;
        }
      }
  };

  if (STAB) {
    // ---- scalar-table walker: one continuous stream of pairs over the range. The
    // loads issued while the last pair of a sequence computes are the next sequence's
    // first pair and query rows, so the pipeline never drains at a sequence boundary.
    // Every iteration issues the same loads (targets chosen by scalar selects; with
    // nothing to fetch, zero-size descriptors return zeros without memory traffic),
    // which keeps the vector-memory waits exact.
    const int64_t blk_bytes = p.c_sb * (int64_t)sizeof(T);
    auto seq_ctx = [&](int bb, int kvt_b) {
      ScalarTableCtx t2;
      t2.kplane = (const char*)p.kc;
      t2.vplane = (const char*)p.vc;
      t2.table = (ConstTable)(p.bt + (int64_t)bb * p.bt_stride);
      t2.blk_bytes = blk_bytes;
      t2.tok_bytes = tok_bytes;
      t2.kvt = kvt_b;
      return t2;
    };
    auto seq_kvt = [&](int bb) {
      const int cx = __builtin_amdgcn_readfirstlane(kv_len(p, bb));
      return seq_kv_tokens(p, cx);
    };
    // this lane's query row of sequence bb: (row ok, token j, query head)
    auto seq_rows = [&](int bb, int& qlen_b, int64_t& qoff_b, bool& ok_b, int& j_b, int& hq_b) {
      seq_queries(p, bb, qlen_b, qoff_b);
      qlen_b = __builtin_amdgcn_readfirstlane(qlen_b);
      const int R = qlen_b * p.n_rep;
      ok_b = n < R;
      j_b = ok_b ? n / p.n_rep : 0;
      hq_b = h * p.n_rep + (ok_b ? n - j_b * p.n_rep : 0);
    };
    // query operand loads through a descriptor over the sequence's query rows (none
    // when !live, rows of lanes with !row_live read as zero). The descriptor is kept
    // wave-uniform (base and size through readfirstlane, the rows masked after the
    // load): a per-lane descriptor makes the compiler wrap every load in a waterfall
    // loop, issued once per distinct descriptor.
    auto load_q = [&](int bb, int64_t qoff_b, int j_b, int hq_b, bool live, bool row_live,
                      u32x4 (&qo)[Tile::KS]) {
      const uint64_t qa = (uint64_t)((const T*)p.q + (int64_t)bb * p.q_sb + qoff_b * p.q_st);
      const char* qb = (const char*)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(qa >> 32)) << 32) |
                                     (uint32_t)__builtin_amdgcn_readfirstlane((int)qa));
      const int qv = (int)(((int64_t)j_b * p.q_st + (int64_t)hq_b * p.q_sh) * (int64_t)sizeof(T)) + 16 * g;
      const __amdgpu_buffer_rsrc_t rq = tile_rsrc(qb, __builtin_amdgcn_readfirstlane(live ? 0x7fffffff : 0));
      const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int s2 = 0; s2 < Tile::KS; ++s2) {
        const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq, qv + 64 * s2, 0, 0));
        qo[s2] = row_live ? v : zero;
      }
    };

    int qlen, j, hq;
    int64_t qoff;
    bool row_ok;
    seq_rows(b, qlen, qoff, row_ok, j, hq);
    int nbp = __builtin_amdgcn_readfirstlane(decode_pairs(p, b));
    int kvt = seq_kvt(b);
    ScalarTableCtx tc = seq_ctx(b, kvt);
    u32x4 qop[Tile::KS], qn[Tile::KS];
    load_q(b, qoff, j, hq, true, true, qop);
    DecodeTile<T, D> ta, tb;
    int pha[2], phb[2], phn[2];
    fetch_phys(p, tc, pos - c, pha);
    load_pair_scalar<T, D, AUX>(p, tc, pos - c, pha, voff_k, voff_v, ta);
    while (true) {
      const int seg0 = pos - c;
      const int seg1 = min(e_w - c, nbp);
      // the next sequence with pairs in this range, if any
      int nb = b + 1;
      bool has_next = c + nbp < e_w;
      if (has_next) {
        while (nb < p.batch && __builtin_amdgcn_readfirstlane(decode_pairs(p, nb)) == 0) ++nb;
        has_next = nb < p.batch;
      }
      int qlen_n = 0, j_n = 0, hq_n = 0, nbp_n = 0, kvt_n = 0;
      int64_t qoff_n = 0;
      bool ok_n = false;
      ScalarTableCtx tcn = tc;
      phn[0] = phn[1] = -1;
      if (has_next) {
        seq_rows(nb, qlen_n, qoff_n, ok_n, j_n, hq_n);
        nbp_n = __builtin_amdgcn_readfirstlane(decode_pairs(p, nb));
        kvt_n = seq_kvt(nb);
        tcn = seq_ctx(nb, kvt_n);
        fetch_phys(p, tcn, 0, phn);
      }
      const int lim = row_ok ? __builtin_amdgcn_readfirstlane(kv_len(p, b)) - qlen + j + 1 : 0;
      const int lim_eff = lim < kvt ? lim : kvt;
      int lim_min = row_ok ? lim_eff : 0x7fffffff;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) lim_min = min(lim_min, __shfl_xor(lim_min, o));
      lim_min = __builtin_amdgcn_readfirstlane(lim_min);

      RowState<T, D> st;
#pragma unroll
      for (int a2 = 0; a2 < RowState<T, D>::NACC; ++a2) st.acc[a2] = f32x4{0.f, 0.f, 0.f, 0.f};
      st.m = kNegBig;
      st.l = 0.f;
      fetch_phys(p, tc, seg0 + 1, phb);

      // prefetch for the pair after pi: the sequence's next pair, else the next
      // sequence's first pair and query rows, else nothing
      auto prefetch = [&](int pi_, const int (&ph_in)[2], DecodeTile<T, D>& dst) {
        const bool in_seg = pi_ + 1 < seg1;
        const bool look = !in_seg && has_next;
        ScalarTableCtx tg = in_seg ? tc : tcn;
        int ph[2];
        ph[0] = in_seg ? ph_in[0] : (look ? phn[0] : -1);
        ph[1] = in_seg ? ph_in[1] : (look ? phn[1] : -1);
        load_pair_scalar<T, D, AUX>(p, tg, in_seg ? pi_ + 1 : 0, ph, voff_k, voff_v, dst);
        load_q(look ? nb : b, look ? qoff_n : qoff, look ? j_n : j, look ? hq_n : hq, look, ok_n, qn);
      };

      int pi = seg0;
      bool next_in_b = false;
      while (true) {
        prefetch(pi, phb, tb);
        __builtin_amdgcn_sched_barrier(0);
        fetch_phys(p, tc, pi + 2, pha);
        compute_pair<T, D>(p, ta, qop, pi, lim_eff, lim_min, lane, st);
        if (++pi >= seg1) {
          next_in_b = true;
          break;
        }
        prefetch(pi, pha, ta);
        __builtin_amdgcn_sched_barrier(0);
        fetch_phys(p, tc, pi + 2, phb);
        compute_pair<T, D>(p, tb, qop, pi, lim_eff, lim_min, lane, st);
        if (++pi >= seg1) break;
      }
      finish(b, c, qoff, j, hq, row_ok, seg0, seg1, nbp, st);
      if (!has_next) break;
      // advance: the next sequence's first pair is already in flight
      pos = c + seg1;
      c += nbp;
      b = nb;
      qlen = qlen_n;
      qoff = qoff_n;
      row_ok = ok_n;
      j = j_n;
      hq = hq_n;
      nbp = nbp_n;
      kvt = kvt_n;
      tc = tcn;
#pragma unroll
      for (int s2 = 0; s2 < Tile::KS; ++s2) qop[s2] = ok_n ? qn[s2] : u32x4{0u, 0u, 0u, 0u};
      if (next_in_b) ta = tb;
    }
  } else {
    while (pos < e_w && b < p.batch) {
      int qlen;
      int64_t qoff;
      seq_queries(p, b, qlen, qoff);
      qlen = __builtin_amdgcn_readfirstlane(qlen);
      const int nbp = __builtin_amdgcn_readfirstlane(decode_pairs(p, b));
      if (nbp == 0) {
        ++b;
        continue;
      }
      const int seg0 = pos - c;
      const int seg1 = min(e_w - c, nbp);
      const int ctx = __builtin_amdgcn_readfirstlane(kv_len(p, b));
      const int kvt = seq_kv_tokens(p, ctx);
      const int R = qlen * p.n_rep;
      const bool row_ok = n < R;
      const int j = row_ok ? n / p.n_rep : 0;
      const int hq = h * p.n_rep + (row_ok ? n - j * p.n_rep : 0);
      const int lim = row_ok ? ctx - qlen + j + 1 : 0;
      const int lim_eff = lim < kvt ? lim : kvt;
      // smallest key limit over this wave's rows: pairs ending before it need no mask
      int lim_min = row_ok ? lim_eff : 0x7fffffff;
  #pragma unroll
      for (int o = 1; o < 64; o <<= 1) lim_min = min(lim_min, __shfl_xor(lim_min, o));
      lim_min = __builtin_amdgcn_readfirstlane(lim_min);
      const T* qrow = (const T*)p.q + (int64_t)b * p.q_sb + (qoff + j) * p.q_st + (int64_t)hq * p.q_sh;
      u32x4 qop[Tile::KS];
  #pragma unroll
      for (int s = 0; s < Tile::KS; ++s) {
        const u32x4 z = {0u, 0u, 0u, 0u};
        qop[s] = row_ok ? load16(qrow + 32 * s + 8 * g) : z;
      }
      const int32_t* table = p.bt + (int64_t)b * p.bt_stride;

      RowState<T, D> st;
  #pragma unroll
      for (int a = 0; a < RowState<T, D>::NACC; ++a) st.acc[a] = f32x4{0.f, 0.f, 0.f, 0.f};
      st.m = kNegBig;
      st.l = 0.f;

      // two-stage software pipeline: loads of pair pi+1 are in flight while pair pi computes
      DecodeTile<T, D> ta, tb;
      int pi = seg0;
      {
        load_pair<T, D>(p, table, kvt, seg0, h, lane, ta);
        while (true) {
          load_pair<T, D>(p, table, kvt, pi + 1, h, lane, tb);
          compute_pair<T, D>(p, ta, qop, pi, lim_eff, lim_min, lane, st);
          if (++pi >= seg1) break;
          load_pair<T, D>(p, table, kvt, pi + 1, h, lane, ta);
          compute_pair<T, D>(p, tb, qop, pi, lim_eff, lim_min, lane, st);
          if (++pi >= seg1) break;
        }
      }

      finish(b, c, qoff, j, hq, row_ok, seg0, seg1, nbp, st);
      pos = c + seg1;
      c += nbp;
      ++b;
    }
  }
  if (rec_writer) {
    rec[0] = rec_b;
    rec[1] = rec_cb;
    rec[2] = rec_cb1;
    rec[3] = rec_slot;
    rec[4] = chunk;
    rec[5] = rec_c0;
    rec[6] = rec_c1;
  }
}

template <typename T, int D, bool STAB, int AUX>
__global__ __launch_bounds__(512) void decode_kernel(const AttnParams p) {
  decode_body<T, D, STAB, AUX, false>(p, blockIdx.x);
}

// The same decode with one more workgroup, the last, that builds the tiled prefill's
// work list of the same packed call (plan_work_list): the prefill launched after it
// needs no plan launch of its own, and the list is built beside the decode instead of
// in a one-workgroup launch that holds the GPU on its own (C3: 5.5 us).
template <typename T, int D, bool STAB, int AUX>
__global__ __launch_bounds__(512) void decode_plan_kernel(const AttnParams p, int* __restrict__ work, int qtiles) {
  if (blockIdx.x == gridDim.x - 1) {
    plan_work_list(p, work, qtiles);
    return;
  }
  decode_body<T, D, STAB, AUX, false>(p, blockIdx.x);
}

// Shared-prefix cascade in one launch: workgroups [0, n_pf) run the prefix pass (the
// tiled prefill over the prefix chunks, pp) and the others the suffix decode's ranges
// (ps, scalar-table walker). The two halves need nothing from each other (the merge
// launch after them folds the prefix parts in) and each CU holds one workgroup, so
// they run side by side on disjoint CUs: the latency-bound pieces of both (item
// prologues, the short suffix ranges) overlap instead of adding up, with no
// cross-queue wait of a second stream.
template <typename T, int D, int AUX>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void cascade_kernel(
    const AttnParams pp, const AttnParams ps, const int n_pf) {
  if ((int)blockIdx.x < n_pf)
    prefill_tile_body<T, D>(pp, nullptr, blockIdx.x, n_pf);
  else
    decode_body<T, D, true, AUX, true>(ps, blockIdx.x - n_pf);
}

// Combine the partials of every sequence cut by a range boundary (blocks
// [0, n_wg)); in a shared-prefix call (n_fin = n_wg) finish the sequences each range
// completed (blocks [n_wg, 2 n_wg), apart from the split ones so that neither waits
// for the other's loads); and write the rows no attention kernel of the call writes
// (the last batch blocks, one per sequence):
//  - a decode sequence with no visible key: zeros (the Triton rule, l == 0);
//  - query rows past what this call's kernels cover, which only a packed stream
//    whose sequence is longer than max_query_len has: zeros, and the status word
//    gets kStatusQueryTooLong, so a broken promise never leaves rows unwritten.
// A packed stream whose cu_seqlens run past total_tokens raises kStatusStreamOverrun
// (seq_queries has clamped it); a shared-prefix call whose prefix is longer than a
// sequence raises kStatusPrefixShort (its suffix counts as empty). In a shared-prefix
// call the merge also folds the prefix parts into the rows it writes.
template <typename T, int D>
__device__ __forceinline__ void decode_merge_body(const AttnParams& p, const int n_wg, const int n_fin, const int blk) {
  const int tid = threadIdx.x;
  if (blk >= n_wg + n_fin) {
    const int b = blk - n_wg - n_fin;
    int qlen;
    int64_t qoff;
    seq_queries(p, b, qlen, qoff);
    if (p.cu && tid == 0 && (p.cu[b + 1] > p.total_tokens || p.cu[b] > p.cu[b + 1] || p.cu[b] < 0))
      atomicOr(&g_status, kStatusStreamOverrun);
    if (p.px_n > 0 && tid == 0 && p.ctx_lens[b] < p.ctx_shift) atomicOr(&g_status, kStatusPrefixShort);
    if (qlen <= 0) return;
    const int R = qlen * p.n_rep;
    int covered;  // rows r = j * n_rep + i (per KV head) some kernel writes
    if (is_decode_seq(p, qlen)) {
      if (decode_pairs(p, b) != 0) return;
      if constexpr (D <= 128) {
        if (p.px_n > 0) {  // shared-prefix cascade, no suffix key: the prefix parts alone
          constexpr int DV = D / 8;
          for (int u = tid; u < qlen * p.n_q * DV; u += blockDim.x) {
            const int c = u % DV, jh = u / DV;
            const int j = jh / p.n_q, hq = jh - j * p.n_q;
            float m = kNegBig, l = 0.f;
            f32x4 ov[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
            fold_prefix<T, D, 1, 8>(p, (int64_t)b * p.n_q + hq, 8 * c, m, l, ov);
            const float inv = l > 0.f ? 1.f / l : 0.f;
            if (p.lse && c == 0) p.lse[lse_index(p, b, qoff, j, hq)] = row_lse(m, l);
            T* o = (T*)p.out + (int64_t)b * p.o_sb + (qoff + j) * p.o_st + (int64_t)hq * p.o_sh + 8 * c;
            store16(o, u32x4{Elem<T>::pack2(ov[0][0] * inv, ov[0][1] * inv), Elem<T>::pack2(ov[0][2] * inv, ov[0][3] * inv),
                             Elem<T>::pack2(ov[1][0] * inv, ov[1][1] * inv), Elem<T>::pack2(ov[1][2] * inv, ov[1][3] * inv)});
          }
          return;
        }
      }
      covered = 0;
    } else {
      covered = min(R, p.row_cap);
      if (covered >= R) return;
      if (tid == 0) atomicOr(&g_status, kStatusQueryTooLong);
    }
    const int j0 = covered / p.n_rep;
    const int64_t per_tok = (int64_t)p.n_q * D;
    for (int64_t idx = (int64_t)j0 * per_tok + tid; idx < (int64_t)qlen * per_tok; idx += blockDim.x) {
      const int j = (int)(idx / per_tok);
      const int rem = (int)(idx - (int64_t)j * per_tok);
      const int hq = rem / D, d = rem - hq * D;
      if (j * p.n_rep + hq % p.n_rep < covered) continue;
      T* o = (T*)p.out + (int64_t)b * p.o_sb + (qoff + j) * p.o_st + (int64_t)hq * p.o_sh + d;
      *o = (T)0.f;
      if (p.lse && d == 0) p.lse[lse_index(p, b, qoff, j, hq)] = -__builtin_inff();
    }
    return;
  }
  if constexpr (D <= 128) {
    if (blk >= n_wg) {  // n_fin > 0: shared-prefix cascade
      const int* rec = p.ws_rec + (int64_t)(blk - n_wg) * 8;
      const int hg = (blk - n_wg) % p.n_hgroups;
      const int c0 = rec[5], c1 = rec[6];
      if (c0 >= 0) {
        // shared-prefix cascade: the sequences this range finished (one query token
        // each), completed with the prefix parts; one thread per (sequence, query head
        // of the head group, 8 consecutive d). [c0, c1) spans the first and last
        // sequence the range finished; a sequence between them with no suffix pair
        // (seq_len == prefix tokens) was skipped by the walker, left no state here, and
        // is written by its own per-sequence block from the prefix parts alone (its
        // slot is read here, as every row's is, and not used: the pair count is read
        // beside the state, one memory round trip for both).
        constexpr int DV = D / 8;
        const int hrows = p.hpw * p.n_rep;
        for (int u = tid; u < (c1 - c0) * hrows * DV; u += blockDim.x) {
          const int c = u % DV, t = u / DV;
          const int bb = c0 + t / hrows, hq = hg * hrows + t % hrows;
          const bool live = decode_pairs(p, bb) != 0;
          const int64_t row = (int64_t)bb * p.n_q + hq;
          float m = p.px_seq_ml[row * 2], l = p.px_seq_ml[row * 2 + 1];
          const f32x4* po = reinterpret_cast<const f32x4*>(p.px_seq_o + row * D + 8 * c);
          f32x4 ov[2] = {po[0], po[1]};
          fold_prefix<T, D, 1, 8>(p, row, 8 * c, m, l, ov);
          if (!live) continue;
          const float inv = l > 0.f ? 1.f / l : 0.f;
          if (p.lse && c == 0) p.lse[row] = row_lse(m, l);
          T* o = (T*)p.out + (int64_t)bb * p.o_sb + (int64_t)hq * p.o_sh + 8 * c;
          store16(o, u32x4{Elem<T>::pack2(ov[0][0] * inv, ov[0][1] * inv), Elem<T>::pack2(ov[0][2] * inv, ov[0][3] * inv),
                           Elem<T>::pack2(ov[1][0] * inv, ov[1][1] * inv), Elem<T>::pack2(ov[1][2] * inv, ov[1][3] * inv)});
        }
      }
      return;
    }
  }
  const int* rec = p.ws_rec + (int64_t)blk * 8;
  const int hg = blk % p.n_hgroups;
  const int b = rec[0];
  if (b < 0) return;
  const int cb1 = rec[2], slot0 = rec[3], chunk = rec[4];
  const int wr0 = blk / p.n_hgroups;
  const int wr1 = (cb1 - 1) / chunk;
  int qlen;
  int64_t qoff;
  seq_queries(p, b, qlen, qoff);
  // One thread per (head, query row, 8 consecutive d): each piece's (max, sum) is read
  // once and its partial output with two 16-byte loads; one 16-byte store.
  const int R = qlen * p.n_rep;
  constexpr int DV = D / 8;
  const int np = wr1 - wr0 + 1;
  for (int u = tid; u < p.hpw * R * DV; u += blockDim.x) {
    const int c = u % DV;
    const int hr = u / DV;
    const int wave = hr / R, r = hr - wave * R;
    auto piece = [&](int i) -> int64_t {
      const int wr = wr0 + i;
      const int slot = i == 0 ? slot0 : 0;
      return (((int64_t)(wr * p.n_hgroups + hg) * 2 + slot) * p.hpw + wave) * p.rmax + r;
    };
    // pieces four at a time: every load of a batch is issued before any is used (one
    // memory round trip per batch), then merged into the running (max, sum, output)
    float mmax = kNegBig, lsum = 0.f;
    f32x4 o0 = {0.f, 0.f, 0.f, 0.f}, o1 = {0.f, 0.f, 0.f, 0.f};
    for (int i0 = 0; i0 < np; i0 += 4) {
      float mv[4], lv[4];
      f32x4 a0[4], a1[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t pi = piece(min(i0 + j, np - 1));
        mv[j] = p.ws_ml[pi * 2];
        lv[j] = p.ws_ml[pi * 2 + 1];
        const f32x4* po = reinterpret_cast<const f32x4*>(p.ws_o + pi * D + 8 * c);
        a0[j] = po[0];
        a1[j] = po[1];
      }
      float mx = mmax;
#pragma unroll
      for (int j = 0; j < 4; ++j) mx = i0 + j < np ? fmaxf(mx, mv[j]) : mx;
      const float keep = fast_exp2(mmax - mx);
      lsum *= keep;
      o0 *= keep;
      o1 *= keep;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float f = i0 + j < np ? fast_exp2(mv[j] - mx) : 0.f;
        lsum += lv[j] * f;
        o0 += a0[j] * f;
        o1 += a1[j] * f;
      }
      mmax = mx;
    }
    const int j = r / p.n_rep;
    const int hq = (hg * p.hpw + wave) * p.n_rep + (r - j * p.n_rep);
    if constexpr (D <= 128) {
      if (p.px_n > 0) {  // shared-prefix cascade: fold in the prefix parts of the row
        f32x4 ov[2] = {o0, o1};
        fold_prefix<T, D, 1, 8>(p, (int64_t)b * p.n_q + hq, 8 * c, mmax, lsum, ov);
        o0 = ov[0];
        o1 = ov[1];
      }
    }
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
    if (p.lse && c == 0) p.lse[lse_index(p, b, qoff, j, hq)] = row_lse(mmax, lsum);
    T* o = (T*)p.out + (int64_t)b * p.o_sb + (qoff + j) * p.o_st + (int64_t)hq * p.o_sh + 8 * c;
    store16(o, u32x4{Elem<T>::pack2(o0[0] * inv, o0[1] * inv), Elem<T>::pack2(o0[2] * inv, o0[3] * inv),
                     Elem<T>::pack2(o1[0] * inv, o1[1] * inv), Elem<T>::pack2(o1[2] * inv, o1[3] * inv)});
  }
}

template <typename T, int D>
__global__ __launch_bounds__(512) void decode_merge_kernel(const AttnParams p, int n_wg, int n_fin) {
  decode_merge_body<T, D>(p, n_wg, n_fin, blockIdx.x);
}

// A packed call's tiled prefill (pp, workgroups [0, n_pf) walking the work list) and
// the merge of its decode (pm, the others) in one launch, after the decode launch: the
// two write disjoint rows. The persistent prefill's workgroups finish unevenly (the
// costliest items set the tail) and the merge blocks take the CUs they leave, instead
// of a launch of their own before or after the prefill.
template <typename T, int D>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_merge_kernel(
    const AttnParams pp, const int* __restrict__ work, const int n_pf, const AttnParams pm, const int n_wg) {
  if ((int)blockIdx.x < n_pf)
    prefill_tile_body<T, D>(pp, work, blockIdx.x, n_pf);
  else
    decode_merge_body<T, D>(pm, n_wg, 0, blockIdx.x - n_pf);
}

}  // namespace

// ---- host side -------------------------------------------------------------

// K+V bytes of one layer's pool up to which the page loads keep the default cache
// policy (the MI355X MALL is 256 MB; leave room for the queries and workspace).
constexpr int64_t kMallReuseBytes = 192ll << 20;

// KV heads per workgroup (one wave each): at most four, so a workgroup puts one wave
// on each SIMD of its CU. With one such workgroup per CU the C2 decode measured
// 268.7 us, against 273.9 us for two per CU and 279.6 us for eight-wave workgroups
// (all with the same eight waves of 248 registers per CU or fewer); it also leaves each
// SIMD room for a wave of another kernel.
static int heads_per_wg(int n_kv) {
  for (int d = 4; d >= 1; --d)
    if (n_kv % d == 0) return d;
  return 1;
}

// Decode workgroups: one per CU (the stream-K ranges of all head groups together).
static int decode_resident_wgs() { return ss_host::device_cu_count(); }

// Longest table (keys) a call may have for the small-batch decode kernel.
constexpr int64_t kSmallDecodeKeys = 1024;

// Decode split-K geometry: number of workgroups and bytes of workspace.
struct DecodeGeometry {
  int hpw, n_hgroups, n_ranges, n_wg, rmax;
  int64_t rec_bytes, ml_bytes, o_bytes;
  int64_t total() const { return rec_bytes + ml_bytes + o_bytes; }
};

// n_ranges ranges per head group (0: one workgroup per CU over all head groups)
template <typename T, int D>
static DecodeGeometry decode_geometry(int n_kv, int rmax, int n_ranges = 0) {
  DecodeGeometry g;
  g.hpw = heads_per_wg(n_kv);
  g.n_hgroups = n_kv / g.hpw;
  g.n_ranges = n_ranges > 0 ? n_ranges : decode_resident_wgs() / g.n_hgroups;
  if (g.n_ranges < 1) g.n_ranges = 1;
  g.n_wg = g.n_ranges * g.n_hgroups;
  g.rmax = rmax;
  g.rec_bytes = (int64_t)g.n_wg * 8 * 4;
  g.ml_bytes = (int64_t)g.n_wg * 2 * g.hpw * rmax * 2 * 4;
  g.o_bytes = (int64_t)g.n_wg * 2 * g.hpw * rmax * D * 4;
  return g;
}

static DecodeGeometry geometry_for(int dtype, int head_dim, int n_kv, int rmax) {
  if (dtype == SS_DTYPE_BF16) {
    if (head_dim == 64) return decode_geometry<bf16_t, 64>(n_kv, rmax);
    if (head_dim == 128) return decode_geometry<bf16_t, 128>(n_kv, rmax);
    return decode_geometry<bf16_t, 256>(n_kv, rmax);
  }
  if (head_dim == 64) return decode_geometry<f16_t, 64>(n_kv, rmax);
  if (head_dim == 128) return decode_geometry<f16_t, 128>(n_kv, rmax);
  return decode_geometry<f16_t, 256>(n_kv, rmax);
}

// Bytes the decode part needs for a launch whose longest query is max_query_len.
int64_t decode_workspace_bytes(int dtype, int head_dim, int n_q, int n_kv, int max_query_len) {
  return geometry_for(dtype, head_dim, n_kv, decode_rows_for(max_query_len, n_q / n_kv)).total();
}

template <typename T, int D>
static int launch_decode_typed(AttnParams p, int max_query_len, char* ws, int64_t ws_bytes,
                               hipStream_t stream, int* plan_work, int plan_qtiles, bool* planned,
                               DeferredMerge* defer) {
  if (planned) *planned = false;
  if (defer) defer->n_wg = 0;
  const DecodeGeometry g = decode_geometry<T, D>(p.n_kv, decode_rows_for(max_query_len, p.n_rep));
  if (ws_bytes < g.total()) {
    ss_host::set_error("paged attention: workspace of %lld bytes, decode needs %lld", (long long)ws_bytes,
                       (long long)g.total());
    return SS_ERR_WORKSPACE;
  }
  // small padded decode calls: one workgroup per (sequence, KV head), no merge (see
  // decode_small_kernel): at most two workgroups per CU and tables of at most 1024 keys
  // (four pairs per wave)
  if constexpr (D <= 128) {
    if (!p.cu && p.px_n == 0 && p.row_cap == 0 && p.chunk_tokens == 0 && p.ctx_shift == 0 &&
        (int64_t)p.tq * p.n_rep <= p.rmax && (int64_t)p.max_blocks * p.block_size <= kSmallDecodeKeys &&
        (int64_t)p.batch * p.n_kv <= 2 * (int64_t)decode_resident_wgs()) {
      hipLaunchKernelGGL((decode_small_kernel<T, D>), dim3((unsigned)((int64_t)p.batch * p.n_kv)), dim3(512), 0,
                         stream, p);
      return ss_host::launch_status("paged attention decode (small)");
    }
  }
  // carve: [rec][ml][o]
  p.ws_rec = (int*)ws;
  p.ws_ml = (float*)(ws + g.rec_bytes);
  p.ws_o = (float*)(ws + g.rec_bytes + g.ml_bytes);
  p.hpw = g.hpw;
  p.n_hgroups = g.n_hgroups;
  p.n_ranges = g.n_ranges;
  int n_wg = g.n_wg;  // fewer ranges than the geometry's use a prefix of its workspace
  if (p.range_cap > 0 && p.n_ranges > p.range_cap) {
    p.n_ranges = p.range_cap;
    n_wg = p.n_ranges * g.n_hgroups;
  }
  if (p.rmax != g.rmax) {
    ss_host::set_error("paged attention: decode row split %d != geometry %d", p.rmax, g.rmax);
    return SS_ERR_INVALID;
  }
  // the scalar-table walker needs block_size >= 16 (one block per 16-token tile); at
  // head_dim 256 its two pairs in flight exceed the register file, so it takes the
  // per-lane path there. Pools whose K and V planes of this layer fit the MALL use the
  // default cache policy, so pages shared between sequences are re-read from it.
  const int64_t pool_bytes = 2 * (int64_t)p.num_blocks * p.c_sb * (int64_t)sizeof(T);
  // with a prefill work list to build (a packed call whose prefill runs after this
  // decode), one more workgroup builds it: 64-thread multiples that divide the plan's
  // 1024 buckets
  const bool plan = plan_work && plan_qtiles > 0 && (1024 % (g.hpw * 64)) == 0;
  if (plan && p.block_size >= 16 && D <= 128) {
    if (pool_bytes > kMallReuseBytes)
      hipLaunchKernelGGL((decode_plan_kernel<T, D, true, kNonTemporal>), dim3(n_wg + 1), dim3(g.hpw * 64), 0, stream,
                         p, plan_work, plan_qtiles);
    else
      hipLaunchKernelGGL((decode_plan_kernel<T, D, true, kDefaultPolicy>), dim3(n_wg + 1), dim3(g.hpw * 64), 0,
                         stream, p, plan_work, plan_qtiles);
    if (planned) *planned = true;
  } else if (p.block_size >= 16 && D <= 128 && pool_bytes > kMallReuseBytes)
    hipLaunchKernelGGL((decode_kernel<T, D, true, kNonTemporal>), dim3(n_wg), dim3(g.hpw * 64), 0, stream, p);
  else if (p.block_size >= 16 && D <= 128)
    hipLaunchKernelGGL((decode_kernel<T, D, true, kDefaultPolicy>), dim3(n_wg), dim3(g.hpw * 64), 0, stream,
                       p);
  else
    hipLaunchKernelGGL((decode_kernel<T, D, false, kDefaultPolicy>), dim3(n_wg), dim3(g.hpw * 64), 0, stream,
                       p);
  int st = ss_host::launch_status("paged attention decode");
  if (st != SS_OK) return st;
  // the merge left to the caller's next launch (a packed call's prefill, which then
  // runs it in its spare workgroups); the call's params with the decode's workspace
  if (defer && plan && p.block_size >= 16 && D <= 128 && p.px_n == 0) {  // only with the list built
    defer->p = p;
    defer->n_wg = n_wg;
    return SS_OK;
  }
  // a shared-prefix merge folds S prefix parts into each of its rows' 8-d pieces (28 x
  // 16 per C4 sequence): 512 threads give every piece its own thread
  const int merge_threads = p.px_n > 0 ? 512 : 256;
  hipLaunchKernelGGL((decode_merge_kernel<T, D>), dim3(n_wg + p.batch), dim3(merge_threads), 0, stream, p, n_wg, 0);
  return ss_host::launch_status("paged attention decode merge");
}

// Shared-prefix cascade: the prefix pass (pp: the tiled prefill over the prefix chunks,
// n_pf workgroups walking its work_qtiles items) and the suffix decode (ps) in one
// launch of cascade_kernel, then the decode merge, which folds the prefix parts in.
// Needs the scalar-table walker and the tiled prefill: block_size >= 16, head_dim <= 128.
template <typename T, int D>
static int launch_cascade_typed(const AttnParams& pp, AttnParams ps, int n_pf, char* ws, int64_t ws_bytes,
                                hipStream_t stream) {
  if constexpr (D > 128) {
    ss_host::set_error("shared-prefix cascade: head_dim %d above 128", D);
    return SS_ERR_UNSUPPORTED;
  } else {
    // ps.range_cap ranges per head group, two per decode workgroup
    const DecodeGeometry g = decode_geometry<T, D>(ps.n_kv, decode_rows_for(1, ps.n_rep), ps.range_cap);
    if (ws_bytes < g.total()) {
      ss_host::set_error("shared-prefix cascade: workspace of %lld bytes, decode needs %lld", (long long)ws_bytes,
                         (long long)g.total());
      return SS_ERR_WORKSPACE;
    }
    if (ps.rmax != g.rmax || ps.block_size < 16 || pp.block_size < 16 || n_pf < 1 || ps.px_n < 1 ||
        ps.range_cap < 2 || g.n_wg % 2 != 0) {
      ss_host::set_error("shared-prefix cascade: invalid launch (rows %d / %d, block_size %d, %d prefix workgroups)",
                         ps.rmax, g.rmax, ps.block_size, n_pf);
      return SS_ERR_INVALID;
    }
    ps.ws_rec = (int*)ws;
    ps.ws_ml = (float*)(ws + g.rec_bytes);
    ps.ws_o = (float*)(ws + g.rec_bytes + g.ml_bytes);
    ps.hpw = g.hpw;
    ps.n_hgroups = g.n_hgroups;
    ps.n_ranges = g.n_ranges;
    const int n_wg = g.n_wg;
    const int lds = 6 * TileCfg<T, D>::PLANE;
    const int64_t pool_bytes = 2 * (int64_t)ps.num_blocks * ps.c_sb * (int64_t)sizeof(T);
    const bool nt = pool_bytes > kMallReuseBytes;
    const void* kern = nt ? (const void*)cascade_kernel<T, D, kNonTemporal> : (const void*)cascade_kernel<T, D, kDefaultPolicy>;
    static bool attr_set[2] = {false, false};  // per instantiation; the attribute is process-wide
    if (!attr_set[nt]) {
      if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess) {
        ss_host::set_error("shared-prefix cascade: cannot reserve %d bytes of LDS", lds);
        return SS_ERR_UNSUPPORTED;
      }
      attr_set[nt] = true;
    }
    if (nt)
      hipLaunchKernelGGL((cascade_kernel<T, D, kNonTemporal>), dim3(n_pf + n_wg / 2), dim3(512), lds, stream, pp,
                         ps, n_pf);
    else
      hipLaunchKernelGGL((cascade_kernel<T, D, kDefaultPolicy>), dim3(n_pf + n_wg / 2), dim3(512), lds, stream, pp,
                         ps, n_pf);
    int st = ss_host::launch_status("shared-prefix cascade");
    if (st != SS_OK) return st;
    // blocks: [0, n_wg) split sequences, [n_wg, 2 n_wg) the sequences each range
    // finished, then one per sequence (rows no other block writes)
    hipLaunchKernelGGL((decode_merge_kernel<T, D>), dim3(2 * n_wg + ps.batch), dim3(512), 0, stream, ps, n_wg,
                       n_wg);
    return ss_host::launch_status("shared-prefix cascade merge");
  }
}

// Read (and optionally clear) this device's status word after the work queued on
// `stream` has finished. The read and the clear are one atomic exchange on the device,
// so a bit that a kernel on another stream ORs in meanwhile is never erased unseen (it
// is either in this read or still in the word for the next one); such a kernel's bits
// show up only once it has run.
// The general kernels (paged_general.hip) keep a word of their own; both are taken.
int general_status_take(int clear, hipStream_t stream);
int general_status_value(int* v);

int read_status(int* flags, int clear, hipStream_t stream) {
  hipLaunchKernelGGL(status_take_kernel, dim3(1), dim3(1), 0, stream, clear);
  if (hipGetLastError() != hipSuccess) return SS_ERR_LAUNCH;
  if (general_status_take(clear, stream) != SS_OK) return SS_ERR_LAUNCH;
  if (hipStreamSynchronize(stream) != hipSuccess) return SS_ERR_LAUNCH;
  int v = 0, vg = 0;
  if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_status_seen), sizeof(int), 0, hipMemcpyDeviceToHost) != hipSuccess)
    return SS_ERR_LAUNCH;
  if (general_status_value(&vg) != SS_OK) return SS_ERR_LAUNCH;
  *flags = v | vg;
  return SS_OK;
}

int decode_heads_per_wg(int n_kv) { return heads_per_wg(n_kv); }

// Bytes of the cascade's decode part: n_ranges ranges per head group.
int64_t cascade_decode_bytes(int dtype, int head_dim, int n_kv, int rmax, int n_ranges) {
  if (dtype == SS_DTYPE_BF16) {
    if (head_dim == 64) return decode_geometry<bf16_t, 64>(n_kv, rmax, n_ranges).total();
    return decode_geometry<bf16_t, 128>(n_kv, rmax, n_ranges).total();
  }
  if (head_dim == 64) return decode_geometry<f16_t, 64>(n_kv, rmax, n_ranges).total();
  return decode_geometry<f16_t, 128>(n_kv, rmax, n_ranges).total();
}

int launch_cascade(const AttnParams& pp, const AttnParams& ps, int n_pf, int dtype, int head_dim, char* ws,
                   int64_t ws_bytes, hipStream_t stream) {
  if (dtype == SS_DTYPE_BF16) {
    if (head_dim == 64) return launch_cascade_typed<bf16_t, 64>(pp, ps, n_pf, ws, ws_bytes, stream);
    if (head_dim == 128) return launch_cascade_typed<bf16_t, 128>(pp, ps, n_pf, ws, ws_bytes, stream);
    return launch_cascade_typed<bf16_t, 256>(pp, ps, n_pf, ws, ws_bytes, stream);
  }
  if (head_dim == 64) return launch_cascade_typed<f16_t, 64>(pp, ps, n_pf, ws, ws_bytes, stream);
  if (head_dim == 128) return launch_cascade_typed<f16_t, 128>(pp, ps, n_pf, ws, ws_bytes, stream);
  return launch_cascade_typed<f16_t, 256>(pp, ps, n_pf, ws, ws_bytes, stream);
}

// A packed call's tiled prefill (pp over the work list) together with the decode merge
// deferred by launch_decode (dm), in one launch: prefill_merge_kernel.
template <typename T, int D>
static int launch_prefill_merge_typed(const AttnParams& pp, int max_query_len, const int* work,
                                      const DeferredMerge& dm, hipStream_t stream) {
  const int64_t qtiles = ((int64_t)(max_query_len < 1 ? 1 : max_query_len) * pp.n_rep + 127) / 128;
  const int64_t items = (int64_t)pp.batch * qtiles * pp.n_kv;
  const int64_t cus = ss_host::device_cu_count();
  const int n_pf = (int)(items < cus ? items : cus);
  const int64_t grid = (int64_t)n_pf + dm.n_wg + dm.p.batch;
  if (grid > 0x7fffffff || n_pf < 1) {
    ss_host::set_error("paged attention: prefill + merge grid of %lld workgroups", (long long)grid);
    return SS_ERR_UNSUPPORTED;
  }
  const int lds = 6 * TileCfg<T, D>::PLANE;  // the prefill's K and V rings
  static bool attr_set = false;  // per instantiation; the attribute is process-wide
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)prefill_merge_kernel<T, D>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            lds) != hipSuccess) {
      ss_host::set_error("paged attention prefill + merge: cannot reserve %d bytes of LDS", lds);
      return SS_ERR_UNSUPPORTED;
    }
    attr_set = true;
  }
  hipLaunchKernelGGL((prefill_merge_kernel<T, D>), dim3((unsigned)grid), dim3(512), lds, stream, pp, work, n_pf, dm.p,
                     dm.n_wg);
  return ss_host::launch_status("paged attention prefill + decode merge");
}

int launch_prefill_merge(const AttnParams& pp, int dtype, int head_dim, int max_query_len, const int* work,
                         const DeferredMerge& dm, hipStream_t stream) {
  if (head_dim > 128 || pp.block_size < 16 || !work || dm.n_wg < 1) {
    ss_host::set_error("paged attention prefill + merge: head_dim %d, block size %d", head_dim, pp.block_size);
    return SS_ERR_UNSUPPORTED;
  }
  if (dtype == SS_DTYPE_BF16)
    return head_dim == 64 ? launch_prefill_merge_typed<bf16_t, 64>(pp, max_query_len, work, dm, stream)
                          : launch_prefill_merge_typed<bf16_t, 128>(pp, max_query_len, work, dm, stream);
  return head_dim == 64 ? launch_prefill_merge_typed<f16_t, 64>(pp, max_query_len, work, dm, stream)
                        : launch_prefill_merge_typed<f16_t, 128>(pp, max_query_len, work, dm, stream);
}

int launch_decode(const AttnParams& p, int dtype, int head_dim, int max_query_len, char* ws,
                  int64_t ws_bytes, hipStream_t stream, int* plan_work, int plan_qtiles, bool* planned,
                  DeferredMerge* defer) {
  if (dtype == SS_DTYPE_BF16) {
    if (head_dim == 64) return launch_decode_typed<bf16_t, 64>(p, max_query_len, ws, ws_bytes, stream, plan_work,
                                                   plan_qtiles, planned, defer);
    if (head_dim == 128) return launch_decode_typed<bf16_t, 128>(p, max_query_len, ws, ws_bytes, stream, plan_work,
                                                   plan_qtiles, planned, defer);
    return launch_decode_typed<bf16_t, 256>(p, max_query_len, ws, ws_bytes, stream, plan_work,
                                                   plan_qtiles, planned, defer);
  }
  if (head_dim == 64) return launch_decode_typed<f16_t, 64>(p, max_query_len, ws, ws_bytes, stream, plan_work,
                                                   plan_qtiles, planned, defer);
  if (head_dim == 128) return launch_decode_typed<f16_t, 128>(p, max_query_len, ws, ws_bytes, stream, plan_work,
                                                   plan_qtiles, planned, defer);
  return launch_decode_typed<f16_t, 256>(p, max_query_len, ws, ws_bytes, stream, plan_work,
                                                   plan_qtiles, planned, defer);
}

}  // namespace ss
