// Chunked-prefill paged attention for gfx950 (query tiles of many rows).
//
// Math: slipstream/models/layers/attention.py:64-88 with the packed causal mask
// of attention.py:32-51 (query j of a Tq-token chunk sits at absolute position
// ctx - Tq + j and sees keys [0, ctx - Tq + j]), gathered through the block
// table as in slipstream/kernels/attention_ref.py:42-65; absent blocks are
// masked (slipstream/kernels/triton_paged.py:161-165).
//
// One workgroup = one (sequence, KV head, tile of 64*NT query rows); the rows
// are (query token j, head i of the GQA group), r = j * n_rep + i, so the
// n_rep heads that share a KV head share every K/V tile. Four wavefronts each
// own 16*NT rows. Per 32-key step the workgroup stages the K and V tiles in LDS
// (double buffered, one barrier per step) and every wave runs
//   S^T = K Q^T   (MFMA 16x16x32, A = K from LDS, B = Q^T in registers)
//   online softmax in fp32, exp2 domain
//   O^T += V^T P^T (A = V^T built in registers with v_perm_b32 from eight
//                   16-byte LDS reads, B = P^T straight from the S^T layout).
#include <type_traits>

#include "attention_common.h"


namespace ss {
int64_t prefill_work_bytes(int64_t batch, int n_rep, int max_query_len);
namespace {

__device__ __attribute__((aligned(16))) uint32_t g_zero_row_p[128];

constexpr int kPrefillWaves = 4;
// Slack (log2 units) by which a row's max may exceed the running max before the
// running state is rescaled (tiled prefill kernel).
constexpr float kRescaleSlack = 8.0f;
constexpr int kKeyTile = 32;

template <typename T, int D, int NT>
struct PrefillCfg {
  static constexpr int NCH = D / 8;           // 16-byte chunks per head row
  static constexpr int MT = (NCH + 15) / 16;  // PV product sets
  static constexpr int KS = D / 32;           // QK k-steps
  static constexpr int ROWS = kPrefillWaves * 16 * NT;
  static constexpr int LDROW = D + 8;         // padded LDS row (elements): 16 B skew per key
  static constexpr int LPT = (kKeyTile * NCH) / (kPrefillWaves * 64);  // 16 B chunks per thread per tile
  static constexpr int NACC = MT * 8;
};

template <typename T, int D, int NT>
__global__ __launch_bounds__(256) void prefill_kernel(const AttnParams p) {
  typedef PrefillCfg<T, D, NT> C;
  __shared__ __attribute__((aligned(16))) T s_k[2][kKeyTile][C::LDROW];
  __shared__ __attribute__((aligned(16))) T s_v[2][kKeyTile][C::LDROW];
  __shared__ __attribute__((aligned(16))) int8_t s_ok[2][kKeyTile];

  const int qt = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  int qlen;
  int64_t qoff;
  seq_queries(p, b, qlen, qoff);
  if (qlen <= 0 || is_decode_seq(p, qlen)) return;
  const int R = qlen * p.n_rep;
  const int row0 = qt * C::ROWS;
  if (row0 >= R) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int ctx = kv_len(p, b);
  const int kvt = seq_kv_tokens(p, ctx);
  const int last_row = min(R - 1, row0 + C::ROWS - 1);
  const int kv_end = min(kvt, ctx - qlen + last_row / p.n_rep + 1);
  const int ntiles = kv_end > 0 ? (kv_end + kKeyTile - 1) / kKeyTile : 0;
  const int32_t* table = p.bt + (int64_t)b * p.bt_stride;

  // rows of this lane: column n of row tile nt
  u32x4 qop[NT][C::KS];
  int lim[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int rr = row0 + wave * 16 * NT + 16 * nt + n;
    const bool ok = rr < R;
    const int j = ok ? rr / p.n_rep : 0;
    const int hq = h * p.n_rep + (ok ? rr - j * p.n_rep : 0);
    const int l = ctx - qlen + j + 1;
    lim[nt] = ok ? (l < kvt ? l : kvt) : 0;
    const T* qrow = (const T*)p.q + (int64_t)b * p.q_sb + (qoff + j) * p.q_st + (int64_t)hq * p.q_sh;
#pragma unroll
    for (int s = 0; s < C::KS; ++s) {
      const u32x4 z = {0u, 0u, 0u, 0u};
      qop[nt][s] = ok ? load16(qrow + 32 * s + 8 * g) : z;
    }
  }

  f32x4 acc[NT][C::NACC];
  float mrow[NT], lrow[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
    for (int a = 0; a < C::NACC; ++a) acc[nt][a] = f32x4{0.f, 0.f, 0.f, 0.f};
    mrow[nt] = kNegBig;
    lrow[nt] = 0.f;
  }

  const char* kc = (const char*)p.kc;
  const char* vc = (const char*)p.vc;
  const char* zero = (const char*)g_zero_row_p;
  const int bmask = p.block_size - 1;
  const int64_t hoff = (int64_t)h * p.c_sh;

  u32x4 rk[C::LPT], rv[C::LPT];
  int rok[C::LPT];
  auto fetch = [&](int kt) {
#pragma unroll
    for (int u = 0; u < C::LPT; ++u) {
      const int ci = tid + 256 * u;
      const int key = ci / C::NCH, cc = ci - key * C::NCH;
      const int ka = kt * kKeyTile + key;
      int bi = ka >> p.bs_shift;
      bi = bi < p.max_blocks ? bi : p.max_blocks - 1;
      const int phys = table[bi];
      const bool ok = ka < kv_end && phys >= 0 && phys < p.num_blocks;
      const int64_t off = ((int64_t)phys * p.c_sb + (int64_t)(ka & bmask) * p.c_so + hoff) * (int64_t)sizeof(T);
      const char* kr = ok ? kc + off : zero;
      const char* vr = ok ? vc + off : zero;
      rk[u] = load16(kr + 8 * cc * (int)sizeof(T));
      rv[u] = load16(vr + 8 * cc * (int)sizeof(T));
      rok[u] = ok;
    }
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int u = 0; u < C::LPT; ++u) {
      const int ci = tid + 256 * u;
      const int key = ci / C::NCH, cc = ci - key * C::NCH;
      store16(&s_k[buf][key][8 * cc], rk[u]);
      store16(&s_v[buf][key][8 * cc], rv[u]);
      if (cc == 0) s_ok[buf][key] = (int8_t)rok[u];
    }
  };

  if (ntiles > 0) {
    fetch(0);
    stage(0);
  }
  __syncthreads();
  const float ninf = -__builtin_inff();
  for (int kt = 0; kt < ntiles; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < ntiles) fetch(kt + 1);

    u32x4 ka[2][C::KS];
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int s = 0; s < C::KS; ++s) ka[x][s] = load16(&s_k[buf][16 * x + n][32 * s + 8 * g]);
    int okw[2];
#pragma unroll
    for (int x = 0; x < 2; ++x) okw[x] = *reinterpret_cast<const int*>(&s_ok[buf][16 * x + 4 * g]);

    u32x4 pop[NT];
    const int tb = kt * kKeyTile + 4 * g;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < C::KS; ++s) {
        s0 = Elem<T>::mfma(ka[0][s], qop[nt][s], s0);
        s1 = Elem<T>::mfma(ka[1][s], qop[nt][s], s1);
      }
      float sv[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool v0 = ((okw[0] >> (8 * e)) & 0xff) && tb + e < lim[nt];
        const bool v1 = ((okw[1] >> (8 * e)) & 0xff) && tb + 16 + e < lim[nt];
        sv[e] = v0 ? s0[e] * p.scale_log2 : ninf;
        sv[4 + e] = v1 ? s1[e] * p.scale_log2 : ninf;
      }
      float mx = sv[0];
#pragma unroll
      for (int e = 1; e < 8; ++e) mx = fmaxf(mx, sv[e]);
      mx = max_across_rows(mx);
      const float mnew = fmaxf(mrow[nt], mx);
      const float alpha = fast_exp2(mrow[nt] - mnew);
      float pv[8], ps = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pv[e] = fast_exp2(sv[e] - mnew);
        ps += pv[e];
      }
      lrow[nt] = lrow[nt] * alpha + ps;
      mrow[nt] = mnew;
#pragma unroll
      for (int a = 0; a < C::NACC; ++a) acc[nt][a] *= alpha;
      pop[nt] = u32x4{Elem<T>::pack2(pv[0], pv[1]), Elem<T>::pack2(pv[2], pv[3]),
                      Elem<T>::pack2(pv[4], pv[5]), Elem<T>::pack2(pv[6], pv[7])};
    }

#pragma unroll
    for (int mt = 0; mt < C::MT; ++mt) {
      const int cc = n + 16 * mt;
      const int ccl = cc < C::NCH ? cc : 0;
      u32x4 vv[8];
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) vv[jj] = load16(&s_v[buf][16 * (jj >> 2) + 4 * g + (jj & 3)][8 * ccl]);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        u32x4 a;
        if (i & 1) {
          a[0] = pick_halves<1, 1>(vv[0][i >> 1], vv[1][i >> 1]);
          a[1] = pick_halves<1, 1>(vv[2][i >> 1], vv[3][i >> 1]);
          a[2] = pick_halves<1, 1>(vv[4][i >> 1], vv[5][i >> 1]);
          a[3] = pick_halves<1, 1>(vv[6][i >> 1], vv[7][i >> 1]);
        } else {
          a[0] = pick_halves<0, 0>(vv[0][i >> 1], vv[1][i >> 1]);
          a[1] = pick_halves<0, 0>(vv[2][i >> 1], vv[3][i >> 1]);
          a[2] = pick_halves<0, 0>(vv[4][i >> 1], vv[5][i >> 1]);
          a[3] = pick_halves<0, 0>(vv[6][i >> 1], vv[7][i >> 1]);
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[nt][mt * 8 + i] = Elem<T>::mfma(a, pop[nt], acc[nt][mt * 8 + i]);
      }
    }

    if (kt + 1 < ntiles) stage(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const float lt = sum_across_rows(lrow[nt]);
    const int rr = row0 + wave * 16 * NT + 16 * nt + n;
    if (rr < R) {
      const int j = rr / p.n_rep;
      const int hq = h * p.n_rep + (rr - j * p.n_rep);
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      T* orow = (T*)p.out + (int64_t)b * p.o_sb + (qoff + j) * p.o_st + (int64_t)hq * p.o_sh;
#pragma unroll
      for (int mt = 0; mt < C::MT; ++mt) {
        const int dbase = 128 * mt + 32 * g;
        if (dbase < D) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const f32x4* a = &acc[nt][mt * 8];
            const u32x4 o = {Elem<T>::pack2(a[0][e] * inv, a[1][e] * inv),
                             Elem<T>::pack2(a[2][e] * inv, a[3][e] * inv),
                             Elem<T>::pack2(a[4][e] * inv, a[5][e] * inv),
                             Elem<T>::pack2(a[6][e] * inv, a[7][e] * inv)};
            store16(orow + dbase + 8 * e, o);
          }
        }
      }
    }
  }
}

// ---- tiled prefill (block_size >= 16, head_dim 64 or 128) -------------------
//
// Same math and row order as prefill_kernel; the K/V path is rebuilt for the
// memory system and the instruction mix of CDNA4:
//  - 64-key tiles arrive by direct-to-LDS buffer loads (16 B per lane) into two
//    rings of three tiles (K and V), so every load has two pipeline steps to
//    land. One wave loads the 16 keys of one group (one block: block_size >= 16)
//    through a descriptor over that block's live tokens; keys past the context
//    or in an absent block read as zero without touching memory.
//  - block-table entries are scalar loads fetched one step ahead; a scan of the
//    sequence's table at the start tells whether any entry below the causal end
//    is absent, and only then are per-tile validity bits kept.
//  - K rows sit in LDS with their 16-byte chunks XOR-swizzled by row, so the 16
//    lanes that read one MFMA operand hit 16 different bank groups.
//  - the V^T operand of O^T += V^T P^T comes from ds_read_b64_tr_b16: within
//    each 16-lane group, lane i receives element i%4 of the 8-byte reads of
//    lanes i/4 + 4e (e = 0..3). Lane s of group G reads key 4G + s/4 (+16 for
//    the second read) at d = (D/4) q + 4 (dt ^ (q & 1)), q = s%4, so lane i of
//    the result holds d = (D/4)(i/4) + 4 (dt ^ (i/4 & 1)) + i%4 for keys
//    4G..4G+3 and 16+4G..16+4G+3 -- the key order of the P^T operand taken
//    straight from the S^T accumulator, and a d order that leaves each lane
//    D/4 consecutive outputs of its row. The dt ^ (q & 1) term sends lanes of
//    odd q to the other 8-byte half of their chunk, which keeps the reads free
//    of LDS bank conflicts.
//  - software pipeline: a step runs the QK product of the next tile next to
//    the softmax of the current one (independent work, one branch-free block).
//  - softmax: the max is taken over raw scores and the scale applied inside the
//    exponent's FMA; the row sum is an MFMA of a ones operand with P^T (the same
//    bf16 probabilities the PV product uses); the running state is rescaled only
//    when some row's max grows, and keys are masked only on tiles that reach
//    past a row's causal limit or hold an absent block.
typedef short tr16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) char* LdsBytes;
typedef const __attribute__((address_space(4))) int32_t* ConstTable;

template <typename T, int D>
struct TileCfg {
  static constexpr int KT = 64;                      // keys per tile
  static constexpr int NCH = D / 8;                  // 16-byte chunks per key row
  static constexpr int ROWB = D * (int)sizeof(T);    // bytes per key row
  static constexpr int PLANE = KT * ROWB;            // K (or V) bytes of one stage
  static constexpr int KS = D / 32;                  // QK k-steps
  static constexpr int DT = D / 16;                  // PV d-tiles
  static constexpr int RPI = 64 / NCH;               // key rows per DMA instruction
  static constexpr int NI = 16 / RPI;                // DMA instructions per 16 keys and plane
  static constexpr int SWSH = ROWB >= 256 ? 0 : 1;   // rows sharing one 256-byte bank cycle
};

template <typename T, int D>
__device__ __forceinline__ int chunk_slot(int row, int c) {
  typedef TileCfg<T, D> C;
  return c ^ ((row >> C::SWSH) & (C::NCH - 1));
}

typedef int i32x4 __attribute__((ext_vector_type(4)));

// Buffer descriptor over [base, base + bytes): stride 0, raw addressing; loads
// past `bytes` return zero.
__device__ __forceinline__ i32x4 span_rsrc(const char* base, int bytes) {
  const uint64_t a = (uint64_t)base;
  return i32x4{(int)(uint32_t)a, (int)((uint32_t)(a >> 32) & 0xFFFF), bytes, 0x00020000};
}

// 16 bytes per lane from rsrc + voff straight into LDS at lds + 16 * lane
// (buffer_load_dwordx4 ... lds; M0 holds the LDS destination). Written as asm
// so that the compiler, which cannot tell the pipeline stages apart, adds no
// vmcnt waits of its own before LDS reads: the kernel waits with explicit
// vmcnt counts and a barrier before a stage is read.
// The compiler's hazard recognizer does not look inside the asm, so the asm
// keeps the wait states itself: the descriptor's size is often written by a
// VALU instruction (v_readfirstlane), and a VMEM instruction may read an SGPR a
// VALU instruction wrote only 5 wait states later (one for M0). With fewer, the
// load can take the previous descriptor's size: after an absent block (size 0)
// the first rows of the next group would read as zeros.
__device__ __forceinline__ void dma16(i32x4 rsrc, LdsBytes lds, int voff) {
  const uint32_t m0 = (uint32_t)(uintptr_t)lds;
  asm volatile(
      "s_nop 4\n\t"
      "buffer_load_dwordx4 %0, %1, 0 offen lds"
      :
      : "v"(voff), "s"(rsrc), "{m0}"(m0)
      : "memory");
}

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

extern __shared__ __attribute__((aligned(1024))) char s_tile_stages[];

// Work split: a workgroup covers 128 query rows of one (sequence, KV head) with
// 8 waves; wave w owns rows 16w .. 16w+15 (one MFMA tile) against all 64 keys of
// every tile. Waves 0-3 issue the K loads and waves 4-7 the V loads of 16-key
// group w%4. Registers are capped at two waves per SIMD (256 per lane); wider
// row tiles per wave (which would halve the LDS reads per row) do not fit that
// budget at head_dim 128, and at one wave per SIMD (up to 512 registers: 4 waves
// of 32 rows) the kernel measured slower (189 vs 150 us on the C3 chunks): one
// wave per SIMD hides too little. The LDS (three K tiles, three V tiles) is
// dynamic shared memory: a static size would make the compiler size registers
// for the occupancy that size alone allows.
template <typename T, int D>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_tile_kernel(
    const AttnParams p, const int* __restrict__ work) {
  typedef TileCfg<T, D> C;
  constexpr int NT = 1;              // 16-row MFMA tiles per wave
  constexpr int ROWS = 128;
  constexpr int XS = 4;              // 16-key subtiles of a tile
  constexpr int LPG = C::NI;         // DMA instructions per wave and load group
  // V ring first: the V reads' stage, row and d offsets then all fit the 16-bit
  // immediate offset of the LDS instructions (the K reads use per-lane bases)
  char* const vring = s_tile_stages;                  // V tile j in slot j % 3
  char* const kring = s_tile_stages + 3 * C::PLANE;   // K tile j in slot j % 3

  // Persistent workgroups walk the work list (prefill_plan_kernel: (sequence,
  // 128-row query tile) entries, costliest first; entry e is the n_kv items
  // e * n_kv + h, one per KV head) in snake order: round r takes item r*G + j, or
  // r*G + G-1-j in odd rounds, so a workgroup that drew a long item early draws a
  // short one next.
  // (With p.work_qtiles > 0 the entries are every (sequence, tile) in order, equal in
  // cost up to the last sequence's, and no list is read.)
  const int wq = p.work_qtiles;
  const int total = (wq > 0 ? p.batch * wq : __builtin_amdgcn_readfirstlane(work[0])) * p.n_kv;
  const int G = gridDim.x, wg = blockIdx.x;
  for (int round = 0; round * G < total; ++round) {
    const int idx = round * G + ((round & 1) ? G - 1 - wg : wg);
    if (idx >= total) continue;
    const int entry = idx / p.n_kv;
    const int bq = wq > 0 ? ((entry / wq) << 16) | (entry % wq) : __builtin_amdgcn_readfirstlane(work[1 + entry]);
    [&](const int b, const int qt, const int h) {
  int qlen;
  int64_t qoff;
  seq_queries(p, b, qlen, qoff);
  // uniform values: keep them in scalar registers (descriptors built from values
  // the compiler takes for divergent get waterfall loops around every load)
  qlen = __builtin_amdgcn_readfirstlane(qlen);
  qoff = __builtin_amdgcn_readfirstlane((int)qoff);
  if (qlen <= 0 || is_decode_seq(p, qlen)) return;
  const int R = qlen * p.n_rep;
  const int row0 = qt * ROWS;
  if (row0 >= R) return;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave & 3;  // the 16-key group whose K (waves 0-3) or V (4-7) this wave loads
  const int n = lane & 15, g = lane >> 4;
  const int ctx = __builtin_amdgcn_readfirstlane(kv_len(p, b));
  const int kvt = seq_kv_tokens(p, ctx);
  const int last_row = min(R - 1, row0 + ROWS - 1);
  const int kv_end = p.noncausal ? kvt : min(kvt, ctx - qlen + last_row / p.n_rep + 1);
  const int ntiles = kv_end > 0 ? (kv_end + C::KT - 1) / C::KT : 0;
  const ConstTable table = (ConstTable)(p.bt + (int64_t)b * p.bt_stride);

  // query rows of this lane (column n of row tile nt) and their causal limits;
  // scores are scaled inside the exponent's FMA, which needs a positive scale:
  // a negative one is applied as its magnitude to the negated query (exact)
  u32x4 qop[NT][C::KS];
  int lim[NT];
  const uint32_t qflip = p.scale_log2 < 0.f ? 0x80008000u : 0u;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int rr = row0 + wave * 16 * NT + 16 * nt + n;
    const bool ok = rr < R;
    const int j = ok ? rr / p.n_rep : 0;
    const int hq = h * p.n_rep + (ok ? rr - j * p.n_rep : 0);
    const int l = p.noncausal ? kvt : ctx - qlen + j + 1;
    lim[nt] = ok ? (l < kvt ? l : kvt) : kvt;
    const int64_t qtok = p.q_period > 0 ? (qoff + j) % p.q_period : qoff + j;
    const T* qrow = (const T*)p.q + (int64_t)b * p.q_sb + qtok * p.q_st + (int64_t)hq * p.q_sh;
#pragma unroll
    for (int s = 0; s < C::KS; ++s) {
      const u32x4 z = {0u, 0u, 0u, 0u};
      qop[nt][s] = (ok ? load16(qrow + 32 * s + 8 * g) : z) ^ u32x4{qflip, qflip, qflip, qflip};
    }
  }
  const float cscale = __builtin_fabsf(p.scale_log2);
  // The query operands must be in registers before the first DMA is issued, so that
  // no wait for them lands inside the pipelined loop: the table scan below waits for
  // its own loads, which were issued after these, before its barrier (one round trip
  // for both; a separate wait here cost one more per item).
  // smallest causal limit over the wave's rows (rows past R do not count)
  const int wrow = min(row0 + wave * 16 * NT, R - 1);
  const int wave_lim = p.noncausal ? kvt : min(kvt, ctx - qlen + wrow / p.n_rep + 1);

  const int tok_bytes = (int)(p.c_so * (int64_t)sizeof(T));
  const int64_t blk_bytes = p.c_sb * (int64_t)sizeof(T);
  const int64_t head_off = (int64_t)h * p.c_sh * (int64_t)sizeof(T);
  const char* const kplane = (const char*)p.kc + head_off;
  const char* const vplane = (const char*)p.vc + head_off;
  const int head_tail = tok_bytes - (int)head_off;  // bytes of a token row from this head on
  const int bmask = p.block_size - 1;

  // raw block-table entries of the four 16-key groups of tile t (scalar loads,
  // checked one step later when the tile is issued)
  auto table_row = [&](int t, int (&e)[4]) {
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const int bi = (t * C::KT + 16 * x) >> p.bs_shift;
      e[x] = table[bi < p.max_blocks ? bi : p.max_blocks - 1];
    }
  };
  // bit x set when group x of tile t lives in a valid block
  auto valid_bits = [&](int t, const int (&e)[4]) {
    int bits = 0;
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const int bi = (t * C::KT + 16 * x) >> p.bs_shift;
      bits |= (bi < p.max_blocks && e[x] >= 0 && e[x] < p.num_blocks) ? (1 << x) : 0;
    }
    return bits;
  };
  // DMA of one plane of tile t: this wave fills the 16 rows of group grp (physical
  // block ph, -1 when absent). Issued for every step, also past the last tile: a
  // zero-size descriptor then moves no data, and every step keeps the same
  // number of loads in flight.
  auto issue = [&](int t, int ph, const char* plane, char* dst) {
    const int key0 = t * C::KT + 16 * grp;
    int live = kv_end - key0;
    live = live < 0 ? 0 : (live > 16 ? 16 : live);
    int64_t off = ph >= 0 ? (int64_t)ph * blk_bytes + (int64_t)(key0 & bmask) * tok_bytes : 0;
    off = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(off >> 32)) << 32) |
                    (uint32_t)__builtin_amdgcn_readfirstlane((int)off));
    const int bytes = __builtin_amdgcn_readfirstlane(ph >= 0 && live > 0 ? (live - 1) * tok_bytes + head_tail : 0);
    const i32x4 rs = span_rsrc(plane + off, bytes);
#pragma unroll
    for (int i = 0; i < C::NI; ++i) {
      const int r = C::RPI * i + lane / C::NCH;  // key row within the group
      const int slot = lane % C::NCH;
      const int voff = r * tok_bytes + chunk_slot<T, D>(r, slot) * 16;
      dma16(rs, (LdsBytes)dst + (16 * grp + C::RPI * i) * C::ROWB, voff);
    }
  };

  // running state per row: max (scaled, exp2 domain), the unnormalised output and
  // the row sum. The sum comes from the matrix cores: a ones A-operand times P^T
  // adds the bf16 probabilities the PV product used, in every row of lsum.
  f32x4 acc[NT][C::DT], lsum[NT];
  float mrow[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
    for (int a = 0; a < C::DT; ++a) acc[nt][a] = f32x4{0.f, 0.f, 0.f, 0.f};
    lsum[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    mrow[nt] = kNegBig;
  }
  constexpr uint32_t kOnePair = std::is_same<T, bf16_t>::value ? 0x3F803F80u : 0x3C003C00u;
  const u32x4 ones = {kOnePair, kOnePair, kOnePair, kOnePair};
  const float ninf = -__builtin_inff();

  // Per-lane LDS read pointers into ring slot 0, the same for every tile (the
  // swizzle of K rows 16x + n and of V rows 32kk + r0 (+16) does not depend on
  // x or kk): slot, subtile and row offsets are then instruction immediates.
  LdsBytes kptr[C::KS];
#pragma unroll
  for (int s = 0; s < C::KS; ++s) kptr[s] = (LdsBytes)kring + (n * C::ROWB + chunk_slot<T, D>(n, 4 * s + g) * 16);
  LdsBytes vptr[C::DT];
  {
    const int sl = lane & 15, G = lane >> 4;
    const int r0 = 4 * G + (sl >> 2);
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
      // d-quad of this lane in d-tile dt: (D/4) q + 4 (dt ^ (q & 1)), q = sl & 3.
      // Lanes of odd q read the other 8-byte half of their 16-byte chunk, so the
      // 32 lanes an LDS cycle serves cover all 64 banks once.
      const int q = sl & 3;
      const int dq = (D / 4) * q + 4 * (dt ^ (q & 1));
      vptr[dt] = (LdsBytes)vring + (r0 * C::ROWB + chunk_slot<T, D>(r0, dq >> 3) * 16 + 2 * (dq & 7));
    }
  }

  // S^T of the tile in K ring slot r (A = K rows from LDS, B = Q^T)
  auto qk = [&](int r, f32x4 (&sacc)[NT][XS]) {
#pragma unroll
    for (int x = 0; x < XS; ++x) {
      u32x4 ka[C::KS];
#pragma unroll
      for (int s = 0; s < C::KS; ++s)
        ka[s] = *(const __attribute__((address_space(3))) u32x4*)(kptr[s] + (r * C::PLANE + 16 * x * C::ROWB));
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        sacc[nt][x] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < C::KS; ++s) sacc[nt][x] = Elem<T>::mfma(ka[s], qop[nt][s], sacc[nt][x]);
      }
    }
  };
  // Scores -> probabilities (packed P^T operand) against the new running max, with
  // no branches; MASK selects the masked variant (keys past a row's causal limit
  // or in an absent block). The max is over raw scores; p = exp2(c s - m).
  auto softmax_p = [&](auto mask_tag, int t, int vbits, const f32x4 (&sacc)[NT][XS], float (&mnew)[NT],
                       u32x4 (&pop)[NT][XS / 2]) {
    constexpr bool MASK = decltype(mask_tag)::value;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      float sv[4 * XS];
#pragma unroll
      for (int x = 0; x < XS; ++x)
#pragma unroll
        for (int e = 0; e < 4; ++e) sv[4 * x + e] = sacc[nt][x][e];
      if (MASK) {
        const int kb = t * C::KT + 4 * g;
#pragma unroll
        for (int x = 0; x < XS; ++x)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            sv[4 * x + e] = (((vbits >> x) & 1) && kb + 16 * x + e < lim[nt]) ? sv[4 * x + e] : ninf;
      }
      float mx = sv[0];
#pragma unroll
      for (int i = 1; i < 4 * XS; ++i) mx = fmaxf(mx, sv[i]);
      mx = max_across_rows(mx);
      // the running max is only raised when some row's max outgrew it by more
      // than kRescaleSlack (log2 units): p then stays below 2^kRescaleSlack, and
      // the rescale of the accumulators is rare after the first tiles
      const float mcand = fmaxf(mrow[nt], mx * cscale);
      mnew[nt] = __any(mcand > mrow[nt] + kRescaleSlack) ? mcand : mrow[nt];
      float pv[4 * XS];
#pragma unroll
      for (int i = 0; i < 4 * XS; ++i) pv[i] = fast_exp2(__builtin_fmaf(sv[i], cscale, -mnew[nt]));
#pragma unroll
      for (int kk = 0; kk < XS / 2; ++kk)
        pop[nt][kk] = u32x4{Elem<T>::pack2(pv[8 * kk + 0], pv[8 * kk + 1]), Elem<T>::pack2(pv[8 * kk + 2], pv[8 * kk + 3]),
                            Elem<T>::pack2(pv[8 * kk + 4], pv[8 * kk + 5]), Elem<T>::pack2(pv[8 * kk + 6], pv[8 * kk + 7])};
    }
  };
  // rescale the running state to the new max (only when some row's max grew)
  auto advance = [&](const float (&mnew)[NT]) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if (__any(mnew[nt] > mrow[nt])) {
        const float alpha = fast_exp2(mrow[nt] - mnew[nt]);
        lsum[nt] *= alpha;
#pragma unroll
        for (int a = 0; a < C::DT; ++a) acc[nt][a] *= alpha;
        mrow[nt] = mnew[nt];
      }
    }
  };
  // O^T += V^T P^T from a V tile. The V operands of the next two MFMAs are read before
  // the current MFMA issues (three operand buffers, the order pinned by scheduling
  // fences): left alone, the register allocator gives each operand pair the registers
  // the previous MFMA just consumed, which puts one LDS round trip in front of every
  // MFMA (C3 chunks: 136.9 -> 125.0 us per launch).
  auto pv_product = [&](const u32x4 (&pop)[NT][XS / 2], int r) {
    constexpr int NP = (XS / 2) * C::DT;  // operand pairs (MFMAs of the product)
    auto vread = [&](int i) {
      const int kk = i / C::DT, dt = i % C::DT;
      const int o1 = r * C::PLANE + 32 * kk * C::ROWB;
      const int o2 = o1 + 16 * C::ROWB;
      const tr16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) tr16x4*)(vptr[dt] + o1));
      const tr16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) tr16x4*)(vptr[dt] + o2));
      const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
      return u32x4{l2[0], l2[1], h2[0], h2[1]};
    };
    constexpr int AHEAD = 2;  // operand pairs in flight ahead of the MFMA that issues
    u32x4 ring[AHEAD + 1];
#pragma unroll
    for (int i = 0; i < AHEAD; ++i) ring[i] = vread(i);
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int kk = i / C::DT, dt = i % C::DT;
      if (i + AHEAD < NP) ring[(i + AHEAD) % (AHEAD + 1)] = vread(i + AHEAD);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[nt][dt] = Elem<T>::mfma(ring[i % (AHEAD + 1)], pop[nt][kk], acc[nt][dt]);
      if (dt == C::DT - 1) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) lsum[nt] = Elem<T>::mfma(ones, pop[nt][kk], lsum[nt]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // one tile: QK of the next tile and the softmax of this one in one branch-free
  // block (independent work the scheduler can interleave), then the rescale and PV
  auto tile_step = [&](int t, int vbits, int knext, const f32x4 (&scur)[NT][XS], f32x4 (&snext)[NT][XS],
                       int vslot) {
    float mnew[NT];
    u32x4 pop[NT][XS / 2];
    if (vbits == 0xF && (t + 1) * C::KT <= wave_lim) {
      qk(knext, snext);
      softmax_p(std::false_type{}, t, vbits, scur, mnew, pop);
    } else {
      qk(knext, snext);
      softmax_p(std::true_type{}, t, vbits, scur, mnew, pop);
    }
    advance(mnew);
    pv_product(pop, vslot);
  };

  // Software pipeline. DMA group j (j >= 1) is {K tile j, V tile j-1}; group 0 is
  // K tile 0 alone. Step t computes QK of tile t+1 next to the softmax and PV of
  // tile t, and issues group t+3 = {K t+3, V t+2} into the slots that tiles t and
  // t-1 freed. A step needs group t+1 and lets group t+2 stay in flight: every
  // load has two steps to land. Tile info lives in slot j % 3 (physical block of
  // this wave's group, valid bits of all four groups), written when K tile j is
  // issued.
  //
  // HOLES: the sequence's table has an absent entry below kv_end. Without one
  // (the common case, found by one scan up front) a wave reads only its own
  // group's entry per tile and no tile needs validity bits.
  const bool k_loader = wave < 4, v_loader = wave >= 4;
  bool bad = false;
  for (int i = threadIdx.x; i * p.block_size < kv_end; i += 512) {
    const int v = p.bt[(int64_t)b * p.bt_stride + i];
    bad |= v < 0 || v >= p.num_blocks;
  }
  const bool holes = __syncthreads_or(bad);
  auto pipeline = [&](auto holes_tag) {
    constexpr bool HOLES = decltype(holes_tag)::value;
    int raw[4];
    auto fetch = [&](int t) {
      if (HOLES) {
        table_row(t, raw);
      } else {
        const int bi = (t * C::KT + 16 * grp) >> p.bs_shift;
        raw[0] = table[bi < p.max_blocks ? bi : p.max_blocks - 1];
      }
    };
    auto tile_info = [&](int t, int& ph, int& vb) {
      if (HOLES) {
        vb = valid_bits(t, raw);
        ph = ((vb >> grp) & 1) ? raw[grp] : -1;
      } else {
        vb = 0xF;
        ph = raw[0];
      }
    };
    int ph0, ph1, ph2, vb0, vb1, vb2;
    fetch(0);
    tile_info(0, ph0, vb0);
    if (k_loader) issue(0, ph0, kplane, kring);
    fetch(1);
    tile_info(1, ph1, vb1);
    if (k_loader) issue(1, ph1, kplane, kring + C::PLANE);
    if (v_loader) issue(0, ph0, vplane, vring);
    fetch(2);
    tile_info(2, ph2, vb2);
    if (k_loader) issue(2, ph2, kplane, kring + 2 * C::PLANE);
    if (v_loader) issue(1, ph1, vplane, vring + C::PLANE);
    fetch(3);
    // three score buffers, one per unrolled step: tile t's scores live in s[t % 3]
    f32x4 sa[NT][XS], sb[NT][XS], sc[NT][XS];
    // group 0 landed; groups 1 and 2 may be in flight (a V loader's first load is
    // in group 1, so it waits for the same count)
    wait_vm<2 * LPG>();
    __syncthreads();
    qk(0, sa);
    // K slot of tile t+1 = (t+1) % 3, V slot of tile t = t % 3
    auto step = [&](int t, int r, int& ph_r, int& vb_r, int ph_v, f32x4 (&scur)[NT][XS], f32x4 (&snext)[NT][XS]) {
      wait_vm<LPG>();
      __syncthreads();
      const int vcur = vb_r;  // tile t's bits; slot r now takes tile t+3
      tile_info(t + 3, ph_r, vb_r);
      if (k_loader) issue(t + 3, ph_r, kplane, kring + r * C::PLANE);
      if (v_loader) issue(t + 2, ph_v, vplane, vring + ((r + 2) % 3) * C::PLANE);
      fetch(t + 4);
      tile_step(t, vcur, (r + 1) % 3, scur, snext, r);
    };
    for (int t = 0; t < ntiles; t += 3) {
      step(t, 0, ph0, vb0, ph2, sa, sb);
      if (t + 1 >= ntiles) break;
      step(t + 1, 1, ph1, vb1, ph0, sb, sc);
      if (t + 2 >= ntiles) break;
      step(t + 2, 2, ph2, vb2, ph1, sc, sa);
    }
  };
  if (holes)
    pipeline(std::true_type{});
  else
    pipeline(std::false_type{});
  // no LDS write may land after the workgroup ends
  wait_vm<0>();

  // each lane holds D/4 consecutive outputs of its row: acc[dt][e] is
  // d = (D/4) g + 4 (dt ^ (g & 1)) + e, so 16-byte store w takes d-tiles 2w and
  // 2w+1, swapped for odd g
  const bool swap = g & 1;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const float lt = lsum[nt][0];
    const int rr = row0 + wave * 16 * NT + 16 * nt + n;
    if (rr < R) {
      const int j = rr / p.n_rep;
      const int hq = h * p.n_rep + (rr - j * p.n_rep);
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      if (p.lse && g == 0) p.lse[lse_index(p, b, qoff, j, hq)] = row_lse(mrow[nt], lt);
      T* orow = (T*)p.out + (int64_t)b * p.o_sb + (qoff + j) * p.o_st + (int64_t)hq * p.o_sh + (D / 4) * g;
#pragma unroll
      for (int w = 0; w < C::DT / 2; ++w) {
        const f32x4 x0 = swap ? acc[nt][2 * w + 1] : acc[nt][2 * w];
        const f32x4 x1 = swap ? acc[nt][2 * w] : acc[nt][2 * w + 1];
        const f32x4 o0 = x0 * inv, o1 = x1 * inv;
        const u32x4 o = {Elem<T>::pack2(o0[0], o0[1]), Elem<T>::pack2(o0[2], o0[3]), Elem<T>::pack2(o1[0], o1[1]),
                         Elem<T>::pack2(o1[2], o1[3])};
        store16(orow + 8 * w, o);
      }
    }
  }
    }(bq >> 16, bq & 0xFFFF, idx - entry * p.n_kv);
    // the next item's loads land in LDS slots that other waves may still read
    __syncthreads();
  }
}

// Work list of the tiled prefill: work[0] = entries, work[1 + i] = (b << 16) | qt for
// every (sequence, 128-row query tile) of a prefill sequence, ordered by decreasing
// cost (64-key tiles below the tile's causal end, plus one): a counting sort over
// cost buckets in LDS. Entries of equal cost land in any order; an item's result
// does not depend on the workgroup that computes it.
constexpr int kPlanBuckets = 1024;
__global__ __launch_bounds__(1024) void prefill_plan_kernel(const AttnParams p, int* __restrict__ work,
                                                             int qtiles) {
  __shared__ int s_hist[kPlanBuckets];
  __shared__ int s_base[kPlanBuckets];
  const int tid = threadIdx.x;  // blockDim.x == kPlanBuckets
  s_hist[tid] = 0;
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
  for (int64_t e = tid; e < n_entries; e += blockDim.x) {
    const int c = bucket(e);
    if (c >= 0) atomicAdd(&s_hist[c], 1);
  }
  __syncthreads();
  {  // exclusive scan from the costliest bucket down: thread t takes bucket 1023 - t
    __shared__ int s_wsum[kPlanBuckets / 64];
    const int lane = tid & 63, wave = tid >> 6;
    const int c = kPlanBuckets - 1 - tid;
    int v = s_hist[c];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_up(v, o);
      v += lane >= o ? t : 0;
    }
    if (lane == 63) s_wsum[wave] = v;
    __syncthreads();
    for (int w = 0; w < wave; ++w) v += s_wsum[w];
    s_base[c] = v - s_hist[c];
    if (tid == kPlanBuckets - 1) work[0] = v;
  }
  __syncthreads();
  for (int64_t e = tid; e < n_entries; e += blockDim.x) {
    const int c = bucket(e);
    if (c >= 0) {
      const int b = (int)(e / qtiles), qt = (int)(e - (int64_t)b * qtiles);
      work[1 + atomicAdd(&s_base[c], 1)] = (b << 16) | qt;
    }
  }
}

constexpr int kPrefillNT = 2;

template <typename T, int D>
int launch_prefill_typed(const AttnParams& p, int max_query_len, int* work, int64_t work_bytes, bool planned,
                         hipStream_t stream) {
  if (D <= 128 && p.block_size >= 16) {
    constexpr int rows = 128;
    const int64_t qtiles = ((int64_t)max_query_len * p.n_rep + rows - 1) / rows;
    if (qtiles < 1 || p.batch < 1) return SS_OK;
    if (qtiles > 0xFFFF || p.batch > 0x7FFF || (int64_t)p.batch * qtiles * p.n_kv > 0x7fffffff) {
      ss_host::set_error("paged attention prefill: too many query tiles (%lld per sequence, batch %d)",
                         (long long)qtiles, p.batch);
      return SS_ERR_UNSUPPORTED;
    }
    const int64_t need = p.work_qtiles > 0 ? 0 : prefill_work_bytes(p.batch, p.n_rep, max_query_len);
    if (p.work_qtiles > 0 && p.work_qtiles != qtiles) {
      ss_host::set_error("paged attention prefill: %d implicit query tiles, the launch has %lld", p.work_qtiles,
                         (long long)qtiles);
      return SS_ERR_INVALID;
    }
    if (need > 0 && (!work || work_bytes < need)) {
      ss_host::set_error("paged attention prefill: workspace of %lld bytes for the work list, needs %lld",
                         (long long)work_bytes, (long long)need);
      return SS_ERR_WORKSPACE;
    }
    constexpr int DD = D <= 128 ? D : 128;
    const int lds = 6 * TileCfg<T, DD>::PLANE;
    static bool attr_set = false;  // per instantiation; the attribute is process-wide
    if (!attr_set) {
      if (hipFuncSetAttribute((const void*)prefill_tile_kernel<T, DD>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess) {
        ss_host::set_error("paged attention prefill: cannot reserve %d bytes of LDS", lds);
        return SS_ERR_UNSUPPORTED;
      }
      attr_set = true;
    }
    if (!planned && p.work_qtiles == 0) {
      hipLaunchKernelGGL(prefill_plan_kernel, dim3(1), dim3(kPlanBuckets), 0, stream, p, work, (int)qtiles);
      int st = ss_host::launch_status("paged attention prefill plan");
      if (st != SS_OK) return st;
    }
    // one resident workgroup per CU (the LDS rings take 96 KB); never more than items
    const int64_t items = (int64_t)p.batch * qtiles * p.n_kv;
    const int64_t cus = ss_host::device_cu_count();
    const int grid = (int)(items < cus ? items : cus);
    hipLaunchKernelGGL((prefill_tile_kernel<T, DD>), dim3((unsigned)grid), dim3(512), lds, stream, p,
                       (const int*)work);
    return ss_host::launch_status("paged attention prefill");
  }
  typedef PrefillCfg<T, D, kPrefillNT> C;
  const int64_t rows = (int64_t)max_query_len * p.n_rep;
  const int64_t qtiles = (rows + C::ROWS - 1) / C::ROWS;
  if (qtiles < 1 || p.batch < 1) return SS_OK;
  if (qtiles > 0x7fffffff || p.batch > 65535 || p.n_kv > 65535) {
    ss_host::set_error("paged attention prefill: grid too large (tiles %lld, batch %d)", (long long)qtiles,
                       p.batch);
    return SS_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL((prefill_kernel<T, D, kPrefillNT>), dim3((unsigned)qtiles, p.n_kv, p.batch),
                     dim3(kPrefillWaves * 64), 0, stream, p);
  return ss_host::launch_status("paged attention prefill");
}

}  // namespace

// Query rows per (sequence, KV head) a prefill launch for max_query_len covers: both
// kernels cut the rows into 128-row query tiles.
int64_t prefill_row_cap(int n_rep, int max_query_len) {
  static_assert(PrefillCfg<bf16_t, 128, kPrefillNT>::ROWS == 128, "per-lane prefill tiles hold 128 rows");
  const int64_t rows = (int64_t)(max_query_len < 1 ? 1 : max_query_len) * n_rep;
  return (rows + 127) / 128 * 128;
}

int64_t prefill_work_bytes(int64_t batch, int n_rep, int max_query_len) {
  const int64_t rows = (int64_t)(max_query_len < 1 ? 1 : max_query_len) * n_rep;
  if (rows <= kDecodeRows) return 0;  // no prefill rows
  return 4 * (1 + batch * ((rows + 127) / 128));
}

int launch_prefill(const AttnParams& p, int dtype, int head_dim, int max_query_len, int* work,
                   int64_t work_bytes, hipStream_t stream, bool planned) {
  if (dtype == SS_DTYPE_BF16) {
    if (head_dim == 64) return launch_prefill_typed<bf16_t, 64>(p, max_query_len, work, work_bytes, planned, stream);
    if (head_dim == 128) return launch_prefill_typed<bf16_t, 128>(p, max_query_len, work, work_bytes, planned, stream);
    return launch_prefill_typed<bf16_t, 256>(p, max_query_len, work, work_bytes, planned, stream);
  }
  if (head_dim == 64) return launch_prefill_typed<f16_t, 64>(p, max_query_len, work, work_bytes, planned, stream);
  if (head_dim == 128) return launch_prefill_typed<f16_t, 128>(p, max_query_len, work, work_bytes, planned, stream);
  return launch_prefill_typed<f16_t, 256>(p, max_query_len, work, work_bytes, planned, stream);
}

}  // namespace ss
