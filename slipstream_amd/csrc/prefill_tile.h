// Tiled chunked-prefill attention (block_size >= 16, head_dim 64 or 128): the device
// code of prefill_tile_kernel, shared by the prefill launch (paged_prefill.hip) and
// the shared-prefix cascade launch (paged_decode.hip).
//
// Math: slipstream/models/layers/attention.py:64-88 with the packed causal mask of
// attention.py:32-51, gathered through the block table as in
// slipstream/kernels/attention_ref.py:42-65; absent blocks are masked
// (slipstream/kernels/triton_paged.py:161-165).
#pragma once
#include <type_traits>

#include "attention_common.h"

namespace ss {
namespace {

// Slack (log2 units) by which a row's max may exceed the running max before the
// running state is rescaled.
constexpr float kRescaleSlack = 8.0f;

// ---- tiled prefill (block_size >= 16, head_dim 64 or 128) -------------------
//
// Same math and row order as prefill_kernel (paged_prefill.hip); the K/V path is rebuilt for the
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
// The body of prefill_tile_kernel as workgroup wg of G (the shared-prefix cascade runs
// it in the first G workgroups of a launch whose others run the decode).
template <typename T, int D>
__device__ __forceinline__ void prefill_tile_body(const AttnParams& p, const int* __restrict__ work, const int wg,
                                                  const int G) {
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

}  // namespace
}  // namespace ss
