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
#include "prefill_tile.h"


namespace ss {
int64_t prefill_work_bytes(int64_t batch, int n_rep, int max_query_len);
namespace {

__device__ __attribute__((aligned(16))) uint32_t g_zero_row_p[128];

constexpr int kPrefillWaves = 4;
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

template <typename T, int D>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_tile_kernel(
    const AttnParams p, const int* __restrict__ work) {
  prefill_tile_body<T, D>(p, work, blockIdx.x, gridDim.x);
}

// The tiled prefill's work list (plan_work_list) built by a one-workgroup launch, when
// no decode launch of the same call builds it.
__global__ __launch_bounds__(1024) void prefill_plan_kernel(const AttnParams p, int* __restrict__ work,
                                                             int qtiles) {
  plan_work_list(p, work, qtiles);
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
