// W4A16 linear y = x @ dequant(W)^T for gfx950 (group-wise asymmetric int4 weights,
// 16-bit activations, fp32 accumulation).
//
// Format (slipstream/kernels/quant_ref.py:8-20,45-69,103-116): qweight [N, K/8]
// int32, nibble n of word j of row o = q[o, 8j + n] at bits 4n; scales [N, K/g]
// (fp16, bf16 or fp32); qzeros [N, K/g] int32; w = (q - zero) * scale.
//
// Fast path (bf16/fp16 activations, K % 128 == 0, g % 32 == 0): MFMA 16x16x32,
// A = activation rows, B = weight rows dequantised in registers by the exponent
// trick: a nibble q OR-ed into the mantissa of 2^7 (bf16) or 2^10 (fp16) is
// exactly MAGIC + q, one v_and_or per pair of weights. For each quantisation
// group the MFMA accumulates G = sum_k x (MAGIC + q), and a second MFMA against
// an all-ones B gives X = sum_k x in the same accumulator layout; then
//     sum_k x (q - z) s = s * G - s * (MAGIC + z) * X,
// exact for any zero point. The nibble pairs come out in the order
// (k0,k4),(k1,k5),(k2,k6),(k3,k7) of each word, and every activation fragment is
// permuted the same way in registers (v_perm_b32), so the dot products pair up.
//
// Untiled kernel (w4a16_kernel): a workgroup owns 16*NS weight rows and 16*MT
// activation rows; its KW waves split K into contiguous slices (each wave streams
// its own slice of the rows: coalesced 16-byte loads, the next block in flight
// while the current one computes), and one LDS pass adds the slices in wave
// order. There is no synchronisation between workgroups.
//
// Skinny kernel (w4a16_skinny_kernel, 2 <= m <= 16 and g == 128): the waves of one
// workgroup split K for 16*NS weight rows, activations staged per wave through LDS,
// no partials leave the workgroup. Tiled kernel (w4a16_tile_kernel, m > 16 and
// g % 128 == 0): four waves split 64*NS weight rows and share the activation tile
// through LDS; K is split over workgroups and a second kernel adds the fp32
// partials in range order. Batch 1 takes a bandwidth GEMV. In every case the
// result does not depend on timing.
//
// Generic path (any other shape, fp32 activations): one thread per output,
// fp32 dequant and dot product.
#include <atomic>
#include <cstdlib>

#include "ss_common.h"

namespace ss {
namespace {

struct W4Params {
  const void* x;
  void* out;
  const uint32_t* qw;
  const void* sc;
  const int32_t* qz;
  int64_t x_stride, o_stride;  // elements
  int m, n, k, g, groups, sdt;
  int kw;  // waves (K slices) per workgroup
};

constexpr int kMaxKW = 8;
// Cache policy of the weight loads: non-temporal (every weight is read once per call;
// streaming without cache allocation measured ~14 % more bandwidth on gfx950).
constexpr int kNonTemporal = 2;
// Cache policy sc1 (device scope): a store written through this XCD's L2 to the point of
// device coherence, a load not served by possibly stale lines of this CU's or XCD's caches.
constexpr int kDeviceScope = 16;

// s_waitcnt vmcnt(0): every vector memory operation of this wave, stores included, has
// completed. Inline asm with a memory clobber, so the compiler keeps every load and store
// written before it on this side of the wait (the waitcnt builtin is not a memory
// operation, and the stores it must cover could be sunk past it).
__device__ __forceinline__ void wait_vm0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Arrival count of one output tile's K ranges in a 64-bit word: bits 8.. hold the call's
// tag, bits 0..7 the ranges arrived. A word with another tag (an earlier call, or memory
// never written) counts as zero arrivals, so the workspace needs no initialisation; the
// last range resets the word to zero, which the first compare-and-swap of the next call
// (or of a replayed launch: a captured graph passes the same tag again) expects.
// No cache maintenance: the partials are device-scope stores the caller has waited for
// (vmcnt 0) before it arrives, the count is a device-scope atomic, and the last range
// reads the partials with device-scope loads. (Release/acquire fences at device scope
// write back or invalidate a whole L2 per wave, several times slower.) This relies on
// sc1 stores reaching the point of device coherence before their vmcnt decrements, and
// on sc1 loads not being served by this XCD's possibly stale L2 lines: the gfx950
// memory model's meaning of the agent-scope cache policy bits.
__device__ __forceinline__ bool arrive_last(unsigned long long* word, unsigned long long tag, int ranges) {
  unsigned long long old = 0ull;
  unsigned long long now;
  do {
    const unsigned long long have = (old & ~0xFFull) == tag ? (old & 0xFFull) : 0ull;
    now = tag | (have + 1);
  } while (!__hip_atomic_compare_exchange_weak(word, &old, now, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT));
  if ((int)(now & 0xFFull) != ranges) return false;
  __hip_atomic_store(word, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

template <typename T>
struct W4Elem;
template <>
struct W4Elem<bf16_t> {
  static constexpr uint32_t kMagicPair = 0x43004300u;  // bf16 128.0 in both halves
  static constexpr uint32_t kOnePair = 0x3F803F80u;    // bf16 1.0 in both halves
  static constexpr float kMagic = 128.f;
  static __device__ __forceinline__ float to_f32(uint32_t h) { return __builtin_bit_cast(float, h << 16); }
};
template <>
struct W4Elem<f16_t> {
  static constexpr uint32_t kMagicPair = 0x64006400u;  // fp16 1024.0 in both halves
  static constexpr uint32_t kOnePair = 0x3C003C00u;    // fp16 1.0 in both halves
  static constexpr float kMagic = 1024.f;
  static __device__ __forceinline__ float to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(f16_t, (uint16_t)h);
  }
};

__device__ __forceinline__ float load_scale(const void* s, int64_t i, int sdt) {
  if (sdt == SS_DTYPE_F16) return (float)((const f16_t*)s)[i];
  if (sdt == SS_DTYPE_BF16) return __builtin_bit_cast(float, (uint32_t)((const uint16_t*)s)[i] << 16);
  return ((const float*)s)[i];
}

// Scales read without branching on their dtype around the load (a load inside a
// dtype branch makes the compiler wait for every outstanding load at the join):
// the aligned dword holding scale gi, through a descriptor bounded by the array
// (bytes past its end read as zero), shifted so the scale's bits are the low ones;
// decoded afterwards.
__device__ __forceinline__ uint32_t scale_bits(__amdgpu_buffer_rsrc_t rs, int64_t gi, int esize) {
  const int off = (int)(gi * esize);
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs, off & ~3, 0, 0) >> (8 * (off & 2));
}
__device__ __forceinline__ float decode_scale(uint32_t bits, int sdt) {
  const float f16 = (float)__builtin_bit_cast(f16_t, (uint16_t)(bits & 0xFFFFu));
  const float b16 = __builtin_bit_cast(float, bits << 16);
  return sdt == SS_DTYPE_F16 ? f16 : (sdt == SS_DTYPE_BF16 ? b16 : __builtin_bit_cast(float, bits));
}

// decode_scale without a branch on the dtype (the branches split the loop body into
// blocks, and the compiler then sinks whole folds past them, keeping every stage's
// MFMA partial sums live): all three decodings, merged under uniform bit masks
// (f16_mask / bf16_mask all-ones for that dtype, else zero).
__device__ __forceinline__ float decode_scale_masked(uint32_t bits, uint32_t f16_mask, uint32_t bf16_mask) {
  const uint32_t f16 = __builtin_bit_cast(uint32_t, (float)__builtin_bit_cast(f16_t, (uint16_t)(bits & 0xFFFFu)));
  const uint32_t b16 = bits << 16;
  return __builtin_bit_cast(float, (f16 & f16_mask) | (b16 & bf16_mask) | (bits & ~(f16_mask | bf16_mask)));
}

// Sum over the 16 lanes of a DPP row (every lane of the row gets the total).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_f32<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp_f32<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp_f32<0x141>(x);  // row_half_mirror
  x += dpp_f32<0x140>(x);  // row_mirror
  return x;
}

// A constant held in a VGPR. gfx9 VOP3 instructions take no literal and read at most
// one SGPR, so (w & mask) | magic becomes one v_and_or_b32 only when the magic word
// already sits in a VGPR (the mask goes to the SGPR slot); otherwise it takes a
// v_and and a v_or with literals.
__device__ __forceinline__ uint32_t in_vgpr(uint32_t c) {
  uint32_t v;
  asm volatile("v_mov_b32 %0, %1" : "=v"(v) : "s"(c));
  return v;
}

// Eight nibbles -> eight 16-bit (MAGIC + q) values in the order k0,k4,k1,k5,k2,k6,k3,k7.
__device__ __forceinline__ u32x4 nibbles_to_operand(uint32_t w, uint32_t magic) {
  return u32x4{(w & 0x000F000Fu) | magic, ((w >> 4) & 0x000F000Fu) | magic, ((w >> 8) & 0x000F000Fu) | magic,
               ((w >> 12) & 0x000F000Fu) | magic};
}

// Eight consecutive 16-bit x values -> the same order as nibbles_to_operand.
__device__ __forceinline__ u32x4 permute_x(u32x4 d) {
  return u32x4{pick_halves<0, 0>(d[0], d[2]), pick_halves<1, 1>(d[0], d[2]), pick_halves<0, 0>(d[1], d[3]),
               pick_halves<1, 1>(d[1], d[3])};
}

// acc + a.lo * b.lo + a.hi * b.hi over packed 16-bit pairs, fp32 accumulation
template <typename T>
__device__ __forceinline__ float dot2_acc(uint32_t a, uint32_t b, float acc);
template <>
__device__ __forceinline__ float dot2_acc<bf16_t>(uint32_t a, uint32_t b, float acc) {
  typedef short s16x2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(s16x2, a), __builtin_bit_cast(s16x2, b), acc, false);
}
template <>
__device__ __forceinline__ float dot2_acc<f16_t>(uint32_t a, uint32_t b, float acc) {
  typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h16x2, a), __builtin_bit_cast(h16x2, b), acc, false);
}

// Raw buffer resource over [base, base + bytes): loads past the end return 0, and a
// per-iteration offset rides in the scalar offset, so the loop does no 64-bit
// address arithmetic.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// MT: 16-row activation tiles; NS: 16-row weight tiles; BIT: 128-key iterations
// per pipeline block; WIDE: g % 128 == 0 (one group per iteration, a lane holds 32
// consecutive keys of its row: one 16-byte load), else g % 32 == 0 (one group per
// 32-key MFMA step, 4-byte loads); XLDS: the workgroup's activation rows (all of K,
// permuted) and their per-fold sums are staged in LDS once -- used when they fit;
// otherwise every wave loads its own activation fragments and sums them with an
// all-ones MFMA.
//
// Dynamic LDS: [XLDS: x rows (K + 8 elements each) | fold sums [K/UNIT][16*MT]]
//              [scale table: 16*NS rows x (2*groups + 2) floats, pairs (s, s*(MAGIC+z))]
// and, once every wave is past the main loop, the same bytes again as the
// reduction buffer (kw - 1) x MT*NS x 64 x f32x4.
template <typename T, int MT, int NS, int BIT, bool WIDE, bool XLDS>
__global__ __launch_bounds__(64 * kMaxKW) void w4a16_kernel(const W4Params p) {
  constexpr int UNIT = WIDE ? 128 : 32;  // keys per fold (one quantisation group; 4 per 128-key iteration if !WIDE)
  typedef W4Elem<T> E;
  extern __shared__ __attribute__((aligned(16))) char s_dyn[];

  const int lane = threadIdx.x & 63;
  // wave-uniform by construction; readfirstlane lets the compiler keep everything
  // derived from it (slice bounds, buffer offsets) in SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ln = lane & 15, kg = lane >> 4;
  const int n0 = blockIdx.x * 16 * NS;
  const int m0 = blockIdx.y * 16 * MT;
  const int rows = min(16 * MT, p.m - m0);
  const int iters = p.k >> 7;
  const int per = (iters + p.kw - 1) / p.kw;
  const int it0 = wave * per;
  const int it1 = min(iters, it0 + per);
  const int lrow = p.k + 8;           // LDS row of x, elements (16-byte skew per row)
  const int szrow = 2 * p.groups + 2;  // LDS row of the scale table, floats (8-byte skew per row)
  const uint32_t magic = in_vgpr(E::kMagicPair);

  T* s_x = (T*)s_dyn;
  const size_t x_bytes = XLDS ? (size_t)rows * lrow * sizeof(T) + (size_t)(p.k / UNIT) * 16 * MT * 4 : 0;
  float* s_xs = (float*)(s_dyn + (XLDS ? (size_t)rows * lrow * sizeof(T) : 0));
  float* s_sz = (float*)(s_dyn + x_bytes);
  f32x4* s_red = (f32x4*)s_dyn;  // aliases the tables above, used after a barrier

  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(p.qw, (uint32_t)((int64_t)p.n * p.k / 2));
  int w_off[NS];  // byte offset of this lane's part of its weight row
#pragma unroll
  for (int ns = 0; ns < NS; ++ns) {
    const int r = min(n0 + ns * 16 + ln, p.n - 1);  // rows past N repeat row N-1; never stored
    w_off[ns] = r * (p.k / 2) + (WIDE ? 16 * kg : 4 * kg);
  }

  struct WBlock {
    u32x4 w[NS][BIT];
  };
  struct XBlock {
    u32x4 x[XLDS ? 1 : MT][XLDS ? 1 : BIT][4];
  };

  // Weight loads only (no use), always in range: iterations past the slice reload
  // the slice's last iteration and fold with scale 0.
  auto load_w = [&](int itb, WBlock& wb) {
#pragma unroll
    for (int it = 0; it < BIT; ++it) {
      const int kk = min(itb + it, it1 - 1) << 7;
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) {
        if (WIDE) {
          wb.w[ns][it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, w_off[ns], kk / 2, kNonTemporal));
        } else {
#pragma unroll
          for (int s = 0; s < 4; ++s)
            wb.w[ns][it][s] = __builtin_amdgcn_raw_buffer_load_b32(rw, w_off[ns], kk / 2 + 16 * s, kNonTemporal);
        }
      }
    }
  };

  // The first block's weights go out before the prologue so their latency overlaps it.
  WBlock wa, wb;
  if (it0 < it1) load_w(it0, wa);

  // ---- prologue: scale table (+ activations) into LDS. Eight entries per thread are
  // requested before any is used (branch-free loads: a load inside a dtype branch
  // makes the compiler wait for every outstanding load after it, which serialised
  // the table behind one memory round trip per entry).
  {
    const int esize = p.sdt == SS_DTYPE_F32 ? 4 : 2;
    const __amdgpu_buffer_rsrc_t rsc = buffer_rsrc(p.sc, (uint32_t)((int64_t)p.n * p.groups * esize));
    const __amdgpu_buffer_rsrc_t rzp = buffer_rsrc(p.qz, (uint32_t)((int64_t)p.n * p.groups * 4));
    const int total = 16 * NS * p.groups;
    for (int q0 = threadIdx.x; q0 < total; q0 += 8 * blockDim.x) {
      uint32_t sbits[8];
      int zv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int q = min(q0 + u * (int)blockDim.x, total - 1);
        const int r = q / p.groups, gi = q - r * p.groups;
        const int64_t si = (int64_t)min(n0 + r, p.n - 1) * p.groups + gi;
        sbits[u] = scale_bits(rsc, si, esize);
        zv[u] = __builtin_amdgcn_raw_buffer_load_b32(rzp, (int)(si * 4), 0, 0);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int q = q0 + u * (int)blockDim.x;
        if (q < total) {
          const int r = q / p.groups, gi = q - r * p.groups;
          const float sc = decode_scale(sbits[u], p.sdt);
          s_sz[r * szrow + 2 * gi] = sc;
          s_sz[r * szrow + 2 * gi + 1] = sc * (E::kMagic + (float)zv[u]);  // s * (MAGIC + z)
        }
      }
    }
  }
  if (XLDS) {
    // rows [m0, m0 + rows) of x for all of K, permuted, plus their fold sums
    constexpr int GL = UNIT / 8;  // staging lanes per fold (consecutive lanes)
    const int cols = p.k / 8;
    for (int q = threadIdx.x; q < rows * cols; q += blockDim.x) {
      const int r = q / cols, c = q - r * cols;
      const u32x4 v = load16((const T*)p.x + (int64_t)(m0 + r) * p.x_stride + 8 * c);
      store16(&s_x[r * lrow + 8 * c], permute_x(v));
      float sum = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) sum += E::to_f32(v[j] & 0xFFFFu) + E::to_f32(v[j] >> 16);
#pragma unroll
      for (int o = 1; o < GL; o <<= 1) sum += __shfl_xor(sum, o);
      if (c % GL == 0) s_xs[(c / GL) * 16 * MT + r] = sum;
    }
    // sums of rows past M are 0 (their outputs are never stored)
    for (int q = threadIdx.x; q < (p.k / UNIT) * 16 * MT; q += blockDim.x)
      if (q % (16 * MT) >= rows) s_xs[q] = 0.f;
  }
  __syncthreads();

  // Activation rows past M read row M-1 (a valid address); they only feed output
  // rows past M, which are never stored (each MFMA output row depends on its own
  // input row alone).
  // activation fragments by buffer loads: one uniform descriptor over this
  // workgroup's rows and a 32-bit offset per lane (a 64-bit address per fragment
  // costs register pairs, and their reuse made the loop head wait for the whole
  // weight prefetch)
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(
      (const T*)p.x + (int64_t)m0 * p.x_stride, (uint32_t)(((int64_t)(rows - 1) * p.x_stride + p.k) * sizeof(T)));
  int xrow[MT];  // byte offset of this lane's activation row
  int xl[MT];    // LDS row (XLDS)
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    xrow[mt] = (int)((int64_t)min(mt * 16 + ln, rows - 1) * p.x_stride * (int64_t)sizeof(T));
    xl[mt] = min(mt * 16 + ln, rows - 1) * lrow;
  }

  f32x4 acc[MT][NS];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) acc[mt][ns] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto load_x = [&](int itb, XBlock& xb) {
    if (XLDS) return;
#pragma unroll
    for (int it = 0; it < BIT; ++it) {
      // the iteration's key offset is uniform: it rides in the scalar offset, so the
      // per-lane offsets stay loop-invariant (no vector register is redefined at the
      // loop head, where reusing a register of the weight prefetch forces a full wait)
      const int kk = (min(itb + it, it1 - 1) << 7) * (int)sizeof(T);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int klane = (WIDE ? 32 * kg + 8 * s : 32 * s + 8 * kg) * (int)sizeof(T);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          xb.x[XLDS ? 0 : mt][XLDS ? 0 : it][s] = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, xrow[mt] + klane, kk, 0));
      }
    }
  };

  const u32x4 ones = {E::kOnePair, E::kOnePair, E::kOnePair, E::kOnePair};
  auto compute = [&](int itb, const WBlock& wblk, const XBlock& xb) {
#pragma unroll
    for (int it = 0; it < BIT; ++it) {
      // no branch: an iteration past the slice computes on reloaded data and folds
      // with scale 0 (a branch here lets the compiler sink this block's loads into it)
      const bool live = itb + it < it1;
      const int kk = min(itb + it, it1 - 1) << 7;
      f32x4 G[MT][NS], X[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        X[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) G[mt][ns] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        u32x4 a[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if (XLDS) {
            a[mt] = load16(&s_x[xl[mt] + kk + (WIDE ? 32 * kg + 8 * s : 32 * s + 8 * kg)]);
          } else {
            a[mt] = permute_x(xb.x[XLDS ? 0 : mt][XLDS ? 0 : it][s]);
            X[mt] = Elem<T>::mfma(a[mt], ones, X[mt]);
          }
        }
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) {
          const u32x4 b = nibbles_to_operand(wblk.w[ns][it][s], magic);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) G[mt][ns] = Elem<T>::mfma(a[mt], b, G[mt][ns]);
        }
        if (!WIDE || s == 3) {  // end of a fold unit: fold it into acc
          const int kf = kk + (WIDE ? 0 : 32 * s);
          if (XLDS) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
              X[mt] = *reinterpret_cast<const f32x4*>(&s_xs[(kf / UNIT) * 16 * MT + mt * 16 + 4 * kg]);
          }
          const int gi = kf / p.g;
#pragma unroll
          for (int ns = 0; ns < NS; ++ns) {
            const float2 sz = *reinterpret_cast<const float2*>(&s_sz[(ns * 16 + ln) * szrow + 2 * gi]);
            const float sc = live ? sz.x : 0.f;
            const float cz = live ? sz.y : 0.f;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
              for (int e = 0; e < 4; ++e) acc[mt][ns][e] = fmaf(sc, G[mt][ns][e], fmaf(-cz, X[mt][e], acc[mt][ns][e]));
              G[mt][ns] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
          }
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) X[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
  };

  if (it0 < it1) {
    // Issue order: weights(b), then x(b), then weights(b+1); compute(b) waits for x(b)
    // and so for everything issued before it, never for weights(b+1). The prefetch is
    // unconditional (past the slice it reloads the slice's last iteration) so every
    // path through the loop has the same loads in flight and the waits stay exact.
    // sched_barrier(0): the scheduler keeps each block's loads issued together ahead of
    // its compute instead of spreading them between the MFMAs.
    XBlock xs;
    int itb = it0;
    while (true) {
      load_x(itb, xs);
      load_w(itb + BIT, wb);
      __builtin_amdgcn_sched_barrier(0);
      compute(itb, wa, xs);
      __builtin_amdgcn_sched_barrier(0);
      itb += BIT;
      if (itb >= it1) break;
      load_x(itb, xs);
      load_w(itb + BIT, wa);
      __builtin_amdgcn_sched_barrier(0);
      compute(itb, wb, xs);
      __builtin_amdgcn_sched_barrier(0);
      itb += BIT;
      if (itb >= it1) break;
    }
  }

  // ---- K slices -> one sum, in wave order
  __syncthreads();  // all waves are done with the tables the reduction buffer overlays
  if (wave > 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) s_red[((wave - 1) * MT * NS + mt * NS + ns) * 64 + lane] = acc[mt][ns];
  }
  __syncthreads();
  if (wave != 0) return;
  for (int w = 1; w < p.kw; ++w) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) acc[mt][ns] += s_red[((w - 1) * MT * NS + mt * NS + ns) * 64 + lane];
  }
  // lane holds C[m0 + mt*16 + 4kg + e][n0 + ns*16 + ln]
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) {
      const int n = n0 + ns * 16 + ln;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + mt * 16 + 4 * kg + e;
        if (m < p.m && n < p.n) ((T*)p.out)[(int64_t)m * p.o_stride + n] = (T)acc[mt][ns][e];
      }
    }
}

// Tiled W4A16 GEMM (m >= 2, g % 128 == 0): the activation tile is shared by the
// workgroup through LDS, so each activation element is read from memory once per
// 64*NS weight rows (the kernel above reads it once per 16*NS rows, which made
// activation traffic several times the weight traffic for m >= 16).
//
// A workgroup owns 16*MT activation rows and 16*NS*WV weight rows (WV waves of 16*NS
// rows each, every wave against all 16*MT activation rows) over one range of `kchunk`
// 128-key stages. With several ranges (split K) each writes fp32 partials
// part[z][m][n]; w4a16_splitk_reduce_kernel adds them in range order, or, with arrival
// words (two ranges), the last range of each output tile to finish adds the other's
// partials to its own in the same order, so the result does not depend on timing.
//   - Once per workgroup: the scale table of its rows and range, as pairs
//     (s, s * (MAGIC + z)) in LDS (dynamic shared memory). Per-stage scale loads
//     from memory, 16 scattered words per instruction, took the memory pipeline
//     slots the weight stream needs.
//   - Per stage: the activation stage (16*MT rows x 128 keys) goes through
//     registers into LDS (double buffered), permuted to the nibble order, with each
//     row's sum over the stage (the X term of the fold; g % 128 == 0 puts a stage
//     in one quantisation group). Weights stream straight into registers PF
//     stages ahead: one 16-byte load per lane and 16-row tile, four lanes reading a
//     row's 64 contiguous bytes. Prefetches past the range use an offset past the
//     end of the buffer: they return zeros without touching memory, and the loop
//     needs no branch.
//   - The loop is VALU-bound rather than MFMA- or memory-bound: per stage and wave
//     (MT = NS = 4, the m > 64 tiles when this was measured) 64 MFMAs against about
//     300 VALU instructions -- the nibble
//     unpack (7 per 32-bit word), the fold (2 FMAs per accumulator element) and the
//     activation staging (its row sums as v_dot2 against ones: 48 fewer per stage
//     than converting and adding each value, 124.6 -> 118.5 us for the C5 layer at
//     m = 64, no change at m = 256). With loads and stores taken out it still took 48 us of the
//     4096 x 28672, m = 256 linear's 101 us; prefetching activations PF stages ahead
//     as well changed nothing.
//   - Per 32-key step the MFMA accumulates G = sum x (MAGIC + q) for every
//     (activation tile, weight tile) pair; one fold per stage:
//       acc += s * G - s * (MAGIC + z) * X.
// Every range is a whole number of PF stages (host-checked).
constexpr int kOutOfRange = 0x40000000;  // buffer offset past any operand (< 2^31 bytes)

template <typename T, int MT, int NS, int PF, int WV>
__global__ __launch_bounds__(64 * WV) __attribute__((amdgpu_waves_per_eu(2, 2))) void w4a16_tile_kernel(
    const W4Params p, float* __restrict__ part, unsigned long long* __restrict__ arrivals, unsigned long long tag,
    int kchunk, int ks, int n_tiles, int m_blocks) {
  typedef W4Elem<T> E;
  constexpr int NTHR = 64 * WV;       // threads
  constexpr int TR = 16 * NS * WV;    // weight rows of the workgroup
  constexpr int XC = 256 * MT / NTHR; // activation-stage chunks per thread
  static_assert(XC >= 1 && 256 * MT % NTHR == 0, "every thread stages whole chunks");
  constexpr int BM = 16 * MT;
  constexpr int LROW = 128 + 8;  // LDS row of an activation stage, elements (16-byte skew)
  __shared__ __attribute__((aligned(16))) T s_x[2][BM][LROW];
  __shared__ __attribute__((aligned(16))) float s_sum[2][BM];
  extern __shared__ __attribute__((aligned(16))) char s_dyn[];
  float2* const s_sz = (float2*)s_dyn;  // [TR rows][gr + 1] (s, s*(MAGIC+z))

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ln = lane & 15, kg = lane >> 4;
  // workgroup -> (K range, weight tile, activation tile). Workgroups go to the eight
  // XCDs round robin, so ids 8 apart share an XCD and its L2: the m_blocks activation
  // tiles of one (range, weight tile) pair get ids 8 apart and are dispatched together,
  // and the weight tile they all read comes from that L2 after the first read (in
  // (range, tile, m) order the pairs' m_blocks reads were a whole grid apart and each
  // came from HBM). The ranges of one weight tile are adjacent pairs, so the resident
  // workgroups read whole weight rows. Ids past the last pair (padding of the last group
  // of eight) exit.
  const int blk = blockIdx.x / (8 * m_blocks), within = blockIdx.x - blk * 8 * m_blocks;
  const int pair = blk * 8 + (within & 7);
  if (pair >= ks * n_tiles) return;
  const int zr = pair % ks;
  const int nb = (pair / ks) * TR;       // the workgroup's first weight row
  const int n0 = nb + wave * 16 * NS;   // this wave's
  const int m0 = (within >> 3) * BM;
  const int rows = min(BM, p.m - m0);
  const int i0 = zr * kchunk;
  const int i1 = min(p.k >> 7, i0 + kchunk);
  const int g0 = (i0 << 7) / p.g;                     // first group of the range
  const int gr = (((i1 << 7) - 1) / p.g) - g0 + 1;    // groups in the range
  const int srow = gr + 1;                            // LDS row of the table (skewed)
  const uint32_t magic = in_vgpr(E::kMagicPair);

  // ---- scale table of rows [nb, nb + 64*NS) x groups [g0, g0 + gr), TB entries per
  // thread per batch. The first batch is requested before the weight prologue and
  // stored after it, so the weights do not wait for a table round trip.
  constexpr int TB = 8;
  const int esize = p.sdt == SS_DTYPE_F32 ? 4 : 2;
  const uint32_t f16_mask = p.sdt == SS_DTYPE_F16 ? ~0u : 0u, bf16_mask = p.sdt == SS_DTYPE_BF16 ? ~0u : 0u;
  const __amdgpu_buffer_rsrc_t rsc = buffer_rsrc(p.sc, (uint32_t)((int64_t)p.n * p.groups * esize));
  const __amdgpu_buffer_rsrc_t rzp = buffer_rsrc(p.qz, (uint32_t)((int64_t)p.n * p.groups * 4));
  const int total = TR * gr;
  uint32_t sbits[TB];
  int zv[TB];
  // entry q = (row q / gr, group q % gr). The quotient through a float reciprocal (a
  // 32-bit integer division is some twenty instructions): the table holds at most
  // kTileTableMax / 8 = 5120 entries of at least 64 rows, so q < 5120 and gr <= 80;
  // (q + 0.5) / gr sits at least 0.5 / gr >= 0.006 from an integer, and the two
  // roundings move it by at most q * 2^-23 < 0.001
  const float inv_gr = 1.0f / (float)gr;
  auto table_row = [&](int q) { return (int)(((float)q + 0.5f) * inv_gr); };
  auto table_load = [&](int q0) {
#pragma unroll
    for (int u = 0; u < TB; ++u) {
      const int q = min(q0 + NTHR * u, total - 1);
      const int r = table_row(q), gl = q - r * gr;
      const int si = min(nb + r, p.n - 1) * p.groups + g0 + gl;
      sbits[u] = scale_bits(rsc, si, esize);
      zv[u] = __builtin_amdgcn_raw_buffer_load_b32(rzp, si * 4, 0, 0);
    }
  };
  auto table_store = [&](int q0) {
#pragma unroll
    for (int u = 0; u < TB; ++u) {
      const int q = q0 + NTHR * u;
      if (q < total) {
        const int r = table_row(q), gl = q - r * gr;
        const float sc = decode_scale_masked(sbits[u], f16_mask, bf16_mask);
        s_sz[r * srow + gl] = float2{sc, sc * (E::kMagic + (float)zv[u])};
      }
    }
  };
  table_load(threadIdx.x);

  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(p.qw, (uint32_t)((int64_t)p.n * p.k / 2));
  int w_off[NS], t_row[NS];
#pragma unroll
  for (int ns = 0; ns < NS; ++ns) {
    const int r = min(n0 + ns * 16 + ln, p.n - 1);  // rows past N repeat row N-1; never stored
    w_off[ns] = r * (p.k / 2) + 16 * kg;
    t_row[ns] = (wave * 16 * NS + ns * 16 + ln) * srow;
  }
  auto load_w = [&](int i, u32x4 (&w)[NS]) {
    const int so = i < i1 ? i * 64 : kOutOfRange;
#pragma unroll
    for (int ns = 0; ns < NS; ++ns)
      w[ns] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, w_off[ns], so, kNonTemporal));
  };

  // activation staging: chunk q = threadIdx.x + NTHR u is row q / 16, keys 8 (q % 16)..+7
  // of the stage; rows past M read row M-1 (their outputs are never stored)
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(
      (const T*)p.x + (int64_t)m0 * p.x_stride, (uint32_t)(((int64_t)(rows - 1) * p.x_stride + p.k) * sizeof(T)));
  int x_off[XC];
#pragma unroll
  for (int u = 0; u < XC; ++u) {
    const int q = threadIdx.x + NTHR * u;
    x_off[u] = (int)(((int64_t)min(q >> 4, rows - 1) * p.x_stride + 8 * (q & 15)) * (int64_t)sizeof(T));
  }
  // two activation stages in registers: stage i + 2 is requested while stage i + 1 is
  // still in flight, ahead of that stage's weight loads, so the wait for an activation
  // stage (the vector-memory counter retires in order) never covers weights issued
  // less than two stages earlier
  u32x4 xr[2][XC];
  auto load_x = [&](int i, u32x4 (&dst)[XC]) {
    const int so = i < i1 ? i * 128 * (int)sizeof(T) : kOutOfRange;
#pragma unroll
    for (int u = 0; u < XC; ++u)
      dst[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, x_off[u], so, 0));
  };
  // the chunk's sum as four v_dot2 against a pair of ones (fp32 accumulation): a quarter
  // of the instructions of converting and adding the eight values one by one
  const uint32_t one2 = in_vgpr(E::kOnePair);
  auto stage_x = [&](int buf, const u32x4 (&src)[XC]) {
#pragma unroll
    for (int u = 0; u < XC; ++u) {
      const int q = threadIdx.x + NTHR * u;
      const int r = q >> 4, c = q & 15;
      float sum = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) sum = dot2_acc<T>(src[u][j], one2, sum);
      sum = row16_sum(sum);  // the 16 chunks of row r sit in one DPP row
      store16(&s_x[buf][r][8 * c], permute_x(src[u]));
      // every lane of the row stores the same total: no branch, so the loop body stays
      // one block (a block boundary lets the compiler sink the folds to the loop end,
      // keeping every stage's partial sums live)
      s_sum[buf][r] = sum;
    }
  };

  f32x4 acc[MT][NS];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) acc[mt][ns] = f32x4{0.f, 0.f, 0.f, 0.f};
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int i, int buf, const u32x4 (&w)[NS]) {
    f32x4 G[MT][NS];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x4 a[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) a[mt] = *reinterpret_cast<const u32x4*>(&s_x[buf][mt * 16 + ln][8 * (4 * kg + s)]);
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) {
        const u32x4 b = nibbles_to_operand(w[ns][s], magic);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) G[mt][ns] = Elem<T>::mfma(a[mt], b, s == 0 ? zero4 : G[mt][ns]);
      }
    }
    f32x4 X[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) X[mt] = *reinterpret_cast<const f32x4*>(&s_sum[buf][mt * 16 + 4 * kg]);
    const int gl = ((i << 7) / p.g) - g0;
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) {
      const float2 sz = s_sz[t_row[ns] + gl];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[mt][ns][e] = fmaf(sz.x, G[mt][ns][e], fmaf(-sz.y, X[mt][e], acc[mt][ns][e]));
    }
  };

  // the first two activation stages, then the weight prologue: staging stage i0 waits
  // for its own activations and the scale table, not for PF stages of weights
  load_x(i0, xr[0]);
  load_x(i0 + 1, xr[1]);
  u32x4 ring[PF][NS];
#pragma unroll
  for (int u = 0; u < PF; ++u) load_w(i0 + u, ring[u]);
  table_store(threadIdx.x);
  for (int q0 = threadIdx.x + TB * NTHR; q0 < total; q0 += TB * NTHR) {  // large tables only
    table_load(q0);
    table_store(q0);
  }
  stage_x(0, xr[0]);
  __syncthreads();  // the scale table and the first activation stage
  for (int i = i0; i < i1; i += PF) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {  // PF is even: stage i + u stages from xr[u & 1]
      const int buf = u & 1;
      load_x(i + u + 2, xr[u & 1]);
      __builtin_amdgcn_sched_barrier(0);
      compute(i + u, buf, ring[u]);
      __builtin_amdgcn_sched_barrier(0);
      load_w(i + u + PF, ring[u]);
      __builtin_amdgcn_sched_barrier(0);
      stage_x(buf ^ 1, xr[(u + 1) & 1]);
      __syncthreads();
    }
  }

  // Results through LDS -- the activation stages' bytes, free after the loop's last
  // barrier -- so that each thread writes 16 contiguous bytes of a row (4-byte stores
  // spread over four rows per instruction took ~1.8 us to issue at m = 64), in passes
  // of MTP activation tiles where the whole tile does not fit.
  // lane holds C[m0 + mt*16 + 4kg + e][n0 + ns*16 + ln]
  constexpr int TW = TR;                                         // the workgroup's columns
  constexpr int TROW = TW + 4;                                   // LDS row, floats (skewed)
  constexpr int PR = (int)(sizeof(s_x) / (TROW * sizeof(float))) / 16 * 16;
  constexpr int MTP = PR / 16 < MT ? PR / 16 : MT;               // activation tiles per pass
  static_assert(MTP >= 1, "a 16-row tile of results fits the activation stages");
  float* const s_t = reinterpret_cast<float*>(&s_x[0][0][0]);
  const bool split = ks > 1;
  // with arrival words (two ranges, N % 4 == 0) the last range finishes the tile (below);
  // without, a second kernel adds the partials after this one
  const bool fused = ks == 2 && arrivals != nullptr;
  // 16-byte chunks (four columns of a row) of the tile per thread, per pass and in all:
  // in pass P a thread handles the chunks P * CPP + li of its CPT (chunk i of a thread is
  // q = threadIdx.x + NTHR i of the tile, rows of TW / 4 chunks)
  constexpr int CPP = MTP * NS;
  constexpr int CPT = MT * NS;
  static_assert(MT % MTP == 0 && CPP * NTHR * 4 == MTP * 16 * TW, "passes of whole chunks per thread");
  f32x4 own[CPT];  // this range's partial sums of the thread's chunks (the two-range finish)
  const bool vec_n = p.n % 4 == 0;
  const bool vec_out = vec_n && p.o_stride % 4 == 0 && ((uintptr_t)p.out & 7) == 0;
  // this range's partials: rows [m0, m0 + BM) of range zr, through a descriptor over
  // them (rows past M are never written); device-scope stores when this kernel finishes
  // the tile
  float* const pbase = part + ((int64_t)zr * p.m + m0) * p.n;
  const __amdgpu_buffer_rsrc_t rp = buffer_rsrc(pbase, (uint32_t)((int64_t)rows * p.n * 4));
#pragma unroll
  for (int mt0 = 0; mt0 < MT; mt0 += MTP) {
    if (mt0 > 0) __syncthreads();  // the previous pass has been read
#pragma unroll
    for (int mt = mt0; mt < mt0 + MTP && mt < MT; ++mt)
#pragma unroll
      for (int ns = 0; ns < NS; ++ns)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          s_t[(16 * (mt - mt0) + 4 * kg + e) * TROW + wave * 16 * NS + 16 * ns + ln] = acc[mt][ns][e];
    __syncthreads();
#pragma unroll
    for (int li = 0; li < CPP; ++li) {
      const int q = threadIdx.x + NTHR * li;
      const int rl = q / (TW / 4), c4 = q - rl * (TW / 4);
      const int m = m0 + 16 * mt0 + rl, n = nb + 4 * c4;
      const f32x4 v = *reinterpret_cast<const f32x4*>(&s_t[rl * TROW + 4 * c4]);
      own[(mt0 / MTP) * CPP + li] = v;
      if (m >= p.m || n >= p.n) continue;
      if (split && vec_n) {
        const int off = (int)(((int64_t)(m - m0) * p.n + n) * 4);
        if (fused)
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rp, off, 0, kDeviceScope);
        else
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rp, off, 0, 0);
      } else if (!split && vec_out) {
        T* const o = (T*)p.out + (int64_t)m * p.o_stride + n;
        const T h[4] = {(T)v[0], (T)v[1], (T)v[2], (T)v[3]};
        *reinterpret_cast<u32x2*>(o) = __builtin_bit_cast(u32x2, h);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (n + e >= p.n) break;
          if (split)
            __hip_atomic_store(part + ((int64_t)zr * p.m + m) * p.n + n + e, v[e], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
          else
            ((T*)p.out)[(int64_t)m * p.o_stride + n + e] = (T)v[e];
        }
      }
    }
  }
  if (!fused) return;

  // Two ranges: the last of the tile's two ranges to arrive adds the other's partials to
  // its own (kept in registers) as (0 + p0) + p1 -- the reduce kernel's sums in its order,
  // whichever range arrives last -- and writes the output: one batch of device-scope
  // loads, half the tile's partial bytes, and no second launch
  __shared__ int s_last;
  wait_vm0();        // this thread's partials have reached the point of device coherence
  __syncthreads();   // every thread's, before the count moves
  if (threadIdx.x == 0) s_last = arrive_last(arrivals + (pair / ks) * m_blocks + (within >> 3), tag, ks) ? 1 : 0;
  __syncthreads();
  if (!s_last) return;
  float* const obase = part + ((int64_t)(1 - zr) * p.m + m0) * p.n;  // the other range's rows
  const __amdgpu_buffer_rsrc_t ro = buffer_rsrc(obase, (uint32_t)((int64_t)rows * p.n * 4));
  u32x4 other[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int q = threadIdx.x + NTHR * i;
    const int rl = q / (TW / 4), c4 = q - rl * (TW / 4);
    const int m = m0 + rl, n = nb + 4 * c4;
    const int off = (m < p.m && n < p.n) ? (int)(((int64_t)rl * p.n + n) * 4) : kOutOfRange;
    other[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ro, off, 0, kDeviceScope));
  }
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int q = threadIdx.x + NTHR * i;
    const int rl = q / (TW / 4), c4 = q - rl * (TW / 4);
    const int m = m0 + rl, n = nb + 4 * c4;
    if (m >= p.m || n >= p.n) continue;
    const f32x4 po = __builtin_bit_cast(f32x4, other[i]);
    const f32x4 p0 = zr == 0 ? own[i] : po, p1 = zr == 0 ? po : own[i];
    f32x4 y;
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = (0.f + p0[e]) + p1[e];
    T* const o = (T*)p.out + (int64_t)m * p.o_stride + n;
    if (vec_out) {
      const T h[4] = {(T)y[0], (T)y[1], (T)y[2], (T)y[3]};
      *reinterpret_cast<u32x2*>(o) = __builtin_bit_cast(u32x2, h);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (n + e < p.n) o[e] = (T)y[e];
    }
  }
}

// Eight int4 weights (one word: keys 8j .. 8j + 7 of a row) -> the MFMA B fragment
// T((q - z) * s) in key order, computed as fma(q, s, -z s) in fp32 and rounded once
// to the activation type. (The reference rounds (q - z) * s to the scales' dtype and
// then to the activation dtype, quant_ref.py:112-116,132; with fp16 scales and bf16
// activations the single rounding differs from that double rounding by at most one
// bf16 ulp of a weight.) Per word: two masks, eight byte converts (v_cvt_f32_ubyteN),
// eight FMAs and four packs.
template <typename T>
__device__ __forceinline__ u32x4 dequant_word(uint32_t w, float s, float nzs) {
  // the masks as asm, so that the compiler does not fold each (lo >> 8b) & 0xFF into a
  // 4-bit field extract and lose the byte converts' own byte select
  uint32_t lo, hi;
  asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(lo) : "v"(w));
  asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(hi) : "v"(w >> 4));
  u32x4 r;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const float qa = (float)((lo >> (8 * b)) & 0xFFu), qb = (float)((hi >> (8 * b)) & 0xFFu);
    r[b] = Elem<T>::pack2(fmaf(qa, s, nzs), fmaf(qb, s, nzs));
  }
  return r;
}

// Scale of SD (a dtype code) from its raw bits (the low 16 bits for 16-bit scales).
template <int SD>
__device__ __forceinline__ float scale_from_bits(uint32_t b) {
  if constexpr (SD == SS_DTYPE_F16) return (float)__builtin_bit_cast(f16_t, (uint16_t)(b & 0xFFFFu));
  if constexpr (SD == SS_DTYPE_BF16) return __builtin_bit_cast(float, b << 16);
  return __builtin_bit_cast(float, b);
}

constexpr int kWideMT = 8, kWideNS = 2, kWideWV = 8, kWidePF = 4;

// Buffer loads for the wide kernel, written as asm: the compiler inserts no vmcnt wait
// of its own for them (its count of loads in flight, merged around the loop's back
// edge, made it wait for nearly every prefetched stage at the top of each stage). The
// kernel waits itself, with vm_wait_tied, whose register operands keep every use of a
// loaded value behind the wait. Descriptors are plain SGPR quads over [base, base + bytes):
// offsets past the end read zeros without a memory access.
typedef int i32x4w __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4w wide_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  return i32x4w{(int)(uint32_t)a, (int)((uint32_t)(a >> 32) & 0xFFFF), (int)bytes, 0x00020000};
}
__device__ __forceinline__ u32x4 asm_load_b128_nt(i32x4w rs, int voff, int soff) {
  u32x4 v;
  asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen nt" : "=v"(v) : "v"(voff), "s"(rs), "s"(soff));
  return v;
}
__device__ __forceinline__ uint32_t asm_load_b32(i32x4w rs, int voff) {
  uint32_t v;
  asm volatile("buffer_load_dword %0, %1, %2, 0 offen" : "=v"(v) : "v"(voff), "s"(rs));
  return v;
}
__device__ __forceinline__ uint32_t asm_load_u16(i32x4w rs, int voff) {
  uint32_t v;
  asm volatile("buffer_load_ushort %0, %1, %2, 0 offen" : "=v"(v) : "v"(voff), "s"(rs));
  return v;
}

// 16 bytes per lane from rs + voff + soff straight into LDS at lds + 16 * lane
// (buffer_load_dwordx4 ... lds; M0 holds the LDS destination). The s_nop: M0 is
// written just before by the compiler, and the load may read it one wait state later.
typedef __attribute__((address_space(3))) char* LdsW;
__device__ __forceinline__ void asm_dma_b128(i32x4w rs, LdsW lds, int voff, int soff) {
  const uint32_t m0 = (uint32_t)(uintptr_t)lds;
  asm volatile("s_nop 1\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(rs), "s"(soff), "{m0}"(m0)
               : "memory");
}

// s_waitcnt vmcnt(N) with the registers of one stage's weight loads as operands, so
// that no use of them is scheduled above the wait.
template <int N, int NS>
__device__ __forceinline__ void vm_wait_tied(u32x4 (&w)[NS]) {
  static_assert(NS == 1 || NS == 2 || NS == 4, "operand lists for one, two or four weight tiles");
  static_assert(N >= 0 && N < 16, "vmcnt range of the encoding used");
  if constexpr (NS == 4)
    asm volatile("s_waitcnt vmcnt(%4)" : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]) : "n"(N) : "memory");
  else if constexpr (NS == 2)
    asm volatile("s_waitcnt vmcnt(%2)" : "+v"(w[0]), "+v"(w[1]) : "n"(N) : "memory");
  else
    asm volatile("s_waitcnt vmcnt(%1)" : "+v"(w[0]) : "n"(N) : "memory");
}

// Wide kernel (w4a16_wide_kernel, m > 64 and g == 128): the weights dequantised once
// per wave into bf16/fp16 MFMA operands, each serving a whole 128-row activation tile.
// Workgroup: WV waves (eight: two per SIMD, so one wave's MFMAs run beside the other's
// dequantisation), 16*MT activation rows x 16*NS*WV weight rows; wave w owns the weight
// rows [nb + 16 NS w, + 16 NS) against every activation row of the tile, so no weight is
// dequantised twice inside a workgroup. Per 128-key stage (one quantisation
// group):
//   - each lane loads its 32 keys of each of its NS weight rows (one 16-byte load per
//     16-row tile, four lanes reading a row's 64 contiguous bytes) PF stages ahead (a
//     register ring; loads past the range use an offset past every operand and return
//     zeros without a memory access), and turns each 8-key word into the B fragment
//     T((q - z) s) in registers (dequant_word); every fragment then feeds MT MFMAs.
//     There is no per-group fold on the accumulators and no activation row sums: the
//     scale is inside the operand. The (s, -z s) pairs of the workgroup's rows and
//     range sit in an LDS table filled once (per-stage scale and zero-point loads, 16
//     rows per instruction, cost about a fifth of the time).
//   - the activation stage (16*MT rows x 128 keys) goes straight into LDS by DMA
//     (buffer_load ... lds: lane l of an instruction writes 16 bytes at 16 l), double
//     buffered with one barrier per stage: an instruction brings four whole rows
//     (256 bytes each), 16-byte chunk c of row r at position c ^ (r % 16) of the row,
//     so that the MFMA A-fragment reads (lane m of a 16-lane group: row m, one chunk)
//     hit sixteen distinct positions: no bank conflicts. Stage i + 2 is requested right
//     after the barrier that ends stage i.
//   - one explicit wait per stage (before that barrier): the loads are asm, issued in a
//     fixed order (stage i: the weights of stage i + PF, then after the barrier the
//     activations of stage i + 2), so the wait for the next activation stage (everything
//     but the NS weight loads just issued) also covers the next stage's weights.
//   - inside a stage, the fragment reads and the dequantisation of key step s + 1 are
//     issued before the MFMAs of step s (two register sets).
//   - results through LDS (the activation buffers) as 16-byte row chunks: the output in
//     T, or with ranges > 1 fp32 partials [ks][m][n] that w4a16_splitk_reduce_kernel
//     adds in range order.
// Per stage and wave (MT = 8): 32 NS MFMAs, 4 NS words dequantised (about 23 VALU
// instructions each) and 32 fragment reads.
template <typename T, int MT, int NS, int WV, int SD>
__global__ __launch_bounds__(64 * WV) void w4a16_wide_kernel(const W4Params p, float* __restrict__ part,
                                                             unsigned long long* __restrict__ arrivals,
                                                             unsigned long long tag, int kchunk, int ks, int n_tiles,
                                                             int m_blocks) {
  constexpr int PF = kWidePF;     // weight stages in flight while one computes
  constexpr int NTHR = 64 * WV;   // threads
  constexpr int BM = 16 * MT;     // activation rows of the workgroup
  constexpr int TR = 16 * NS * WV;  // weight rows of the workgroup
  constexpr int XBYTES = BM * 256;  // one activation stage
  constexpr int XI = BM / (4 * WV);  // DMA instructions per wave and stage (four rows each)
  static_assert(XI * 4 * WV == BM, "whole DMA instructions per wave");
  constexpr int ESZ = SD == SS_DTYPE_F32 ? 4 : 2;
  static_assert(PF % 2 == 0, "stage i + u reads activation buffer u & 1");
  extern __shared__ __attribute__((aligned(16))) char s_dyn[];
  float2* const s_tab = reinterpret_cast<float2*>(s_dyn + 2 * XBYTES);  // [stage of the range][TR]

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ln = lane & 15, kg = lane >> 4;
  // workgroup -> (K range, weight tile, activation block), the activation blocks of one
  // (range, weight tile) pair 8 ids apart so that they share an XCD and its L2 (the
  // workgroups go round robin over the eight XCDs); ids past the last pair exit
  const int blk = blockIdx.x / (8 * m_blocks), within = blockIdx.x - blk * 8 * m_blocks;
  const int pair = blk * 8 + (within & 7);
  if (pair >= ks * n_tiles) return;
  const int zr = pair % ks;
  const int nb = (pair / ks) * TR;
  const int n0 = nb + wave * 16 * NS;
  const int m0 = (within >> 3) * BM;
  const int rows = min(BM, p.m - m0);
  const int i0 = zr * kchunk;
  const int i1 = min(p.k >> 7, i0 + kchunk);
  const int nst = i1 - i0;

  // ---- weights: rows past N repeat row N - 1 (never stored)
  const i32x4w rw = wide_rsrc(p.qw, (uint32_t)((int64_t)p.n * p.k / 2));
  int w_off[NS];
#pragma unroll
  for (int ns = 0; ns < NS; ++ns) w_off[ns] = min(n0 + ns * 16 + ln, p.n - 1) * (p.k / 2) + 16 * kg;
  u32x4 wr[PF][NS];
  // The loads are asm, so the compiler's hazard recognizer does not see them read the
  // offset SGPR: a VALU write of an SGPR (v_readfirstlane) needs five wait states before
  // a VMEM instruction reads it. The s_nop, ordered after the offset's computation by its
  // operand and before the loads as a volatile asm, keeps them whatever the schedule.
  auto load_w = [&](int i, u32x4 (&w)[NS]) {
    const int so = __builtin_amdgcn_readfirstlane(i < i1 ? i * 64 : kOutOfRange);
    asm volatile("s_nop 4" : : "s"(so));
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) w[ns] = asm_load_b128_nt(rw, w_off[ns], so);
  };

  // ---- activations: DMA instruction u of wave w brings rows 4 (XI w + u) + l / 16 of
  // the stage, lane l the chunk (l % 16) ^ (row % 16); rows past M read row M - 1 (their
  // outputs are never stored)
  const i32x4w rx = wide_rsrc((const T*)p.x + (int64_t)m0 * p.x_stride,
                              (uint32_t)(((int64_t)(rows - 1) * p.x_stride + p.k) * sizeof(T)));
  int x_off[XI];
#pragma unroll
  for (int u = 0; u < XI; ++u) {
    const int r = 4 * (XI * wave + u) + kg;
    x_off[u] = (int)((int64_t)min(r, rows - 1) * p.x_stride * (int64_t)sizeof(T)) + 16 * (ln ^ (r & 15));
  }
  const LdsW lds_x = (LdsW)s_dyn;
  auto dma_x = [&](int i, int buf) {
    const int so = __builtin_amdgcn_readfirstlane(i < i1 ? i * 128 * (int)sizeof(T) : kOutOfRange);
    asm volatile("s_nop 4" : : "s"(so));  // as in load_w
#pragma unroll
    for (int u = 0; u < XI; ++u) asm_dma_b128(rx, lds_x + buf * XBYTES + (XI * wave + u) * 1024, x_off[u], so);
  };
  // A fragment (tile mt, key step s) of lane (ln, kg): row 16 mt + ln, keys 32 kg + 8 s
  // (the keys of the weight word the lane's B fragment holds in step s), i.e. chunk
  // 4 kg + s of the row, at position (4 kg + s) ^ ln
  int a_off[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) a_off[s] = (ln >> 2) * 1024 + (ln & 3) * 256 + 16 * ((4 * kg + s) ^ ln);

  // ---- the (s, -z s) table of the workgroup's rows over the range's stages, in
  // batches of TB entries per thread; the first batch is requested before the weight and
  // activation prologue, so their latencies overlap
  constexpr int TB = 16;
  const i32x4w rsc = wide_rsrc(p.sc, (uint32_t)((int64_t)p.n * p.groups * ESZ));
  const i32x4w rzp = wide_rsrc(p.qz, (uint32_t)((int64_t)p.n * p.groups * 4));
  const int total = TR * nst;
  uint32_t sb[TB], zb[TB];
  auto table_load = [&](int q0) {
#pragma unroll
    for (int j = 0; j < TB; ++j) {  // entry q: row q / nst, stage q % nst (groups contiguous)
      const int q = min(q0 + NTHR * j + (int)threadIdx.x, total - 1);
      const int r = q / nst, gl = q - r * nst;
      const int gi = min(nb + r, p.n - 1) * p.groups + i0 + gl;
      sb[j] = ESZ == 2 ? asm_load_u16(rsc, gi * 2) : asm_load_b32(rsc, gi * 4);
      zb[j] = asm_load_b32(rzp, gi * 4);
    }
  };
  auto table_tie = [&]() {  // no use of the batch above the preceding wait
    asm volatile("" : "+v"(sb[0]), "+v"(sb[1]), "+v"(sb[2]), "+v"(sb[3]), "+v"(sb[4]), "+v"(sb[5]), "+v"(sb[6]),
                 "+v"(sb[7]), "+v"(sb[8]), "+v"(sb[9]), "+v"(sb[10]), "+v"(sb[11]), "+v"(sb[12]), "+v"(sb[13]),
                 "+v"(sb[14]), "+v"(sb[15]));
    asm volatile("" : "+v"(zb[0]), "+v"(zb[1]), "+v"(zb[2]), "+v"(zb[3]), "+v"(zb[4]), "+v"(zb[5]), "+v"(zb[6]),
                 "+v"(zb[7]), "+v"(zb[8]), "+v"(zb[9]), "+v"(zb[10]), "+v"(zb[11]), "+v"(zb[12]), "+v"(zb[13]),
                 "+v"(zb[14]), "+v"(zb[15]));
  };
  auto table_store = [&](int q0) {
#pragma unroll
    for (int j = 0; j < TB; ++j) {
      const int q = q0 + NTHR * j + (int)threadIdx.x;
      if (q < total) {
        const int r = q / nst, gl = q - r * nst;
        const float sc = scale_from_bits<SD>(sb[j]);
        s_tab[gl * TR + r] = float2{sc, -sc * (float)(int)zb[j]};
      }
    }
  };

  f32x4 acc[MT][NS];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) acc[mt][ns] = f32x4{0.f, 0.f, 0.f, 0.f};

  // One stage: key step s multiplies the fragments read during step s - 1 with the B
  // operands dequantised during step s - 1, while the next step's fragments are read
  // and its weights dequantised.
  auto compute = [&](int i, int buf, const u32x4 (&w)[NS]) {
    float sc[NS], nzs[NS];
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) {
      const float2 t = s_tab[(i - i0) * TR + wave * 16 * NS + 16 * ns + ln];
      sc[ns] = t.x;
      nzs[ns] = t.y;
    }
    const char* const xs = (const char*)s_dyn + buf * XBYTES;
    u32x4 a[2][MT], b[2][NS];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) a[0][mt] = *reinterpret_cast<const u32x4*>(xs + mt * 4096 + a_off[0]);
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) b[0][ns] = dequant_word<T>(w[ns][0], sc[ns], nzs[ns]);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int c = s & 1;
      if (s < 3) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          a[c ^ 1][mt] = *reinterpret_cast<const u32x4*>(xs + mt * 4096 + a_off[s + 1]);
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) b[c ^ 1][ns] = dequant_word<T>(w[ns][s + 1], sc[ns], nzs[ns]);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) acc[mt][ns] = Elem<T>::mfma(a[c][mt], b[c][ns], acc[mt][ns]);
    }
    // One wave per SIMD: the next step's fragment reads and dequantisation only overlap
    // the MFMAs if they are issued between them (in order, a VALU instruction issues
    // while the matrix core works on the MFMA before it). Per step: MT * NS MFMAs, each
    // followed by three VALU instructions, a fragment read before every NS MFMAs.
#pragma unroll
    for (int s = 0; s < 3; ++s)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // VALU
        }
      }
  };

  // prologue: the first table batch, PF weight stages and the first two activation
  // stages requested; all but the second activation stage landed, the table stored
  asm volatile("s_nop 4");  // descriptor SGPRs written by VALU (readfirstlane) before the first load
  table_load(0);
#pragma unroll
  for (int u = 0; u < PF; ++u) load_w(i0 + u, wr[u]);
  dma_x(i0, 0);
  dma_x(i0 + 1, 1);
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(XI) : "memory");
  table_tie();
  vm_wait_tied<0, NS>(wr[0]);  // (no-op by now: register operands only)
  table_store(0);
  for (int q0 = NTHR * TB; q0 < total; q0 += NTHR * TB) {  // tables of more than one batch
    table_load(q0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    table_tie();
    table_store(q0);
  }
  __syncthreads();
  // every range is a whole number of PF stages (host-checked): no branch in the body,
  // which keeps the accumulators in place across the unrolled stages. Stage j reads
  // activation buffer j & 1 (i0 is a multiple of PF, PF is even).
  for (int i = i0; i < i1; i += PF) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      compute(i + u, u & 1, wr[u]);
      load_w(i + u + PF, wr[u]);
      // the activations of stage i + u + 1 (requested before the NS weight loads just
      // issued) and, older, the weights of stage i + u + 1 have landed
      vm_wait_tied<NS, NS>(wr[(u + 1) % PF]);
      __syncthreads();  // every wave's part of stage i + u + 1 is in LDS; buffer u & 1 is free
      dma_x(i + u + 2, u & 1);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // prefetches past the range
  __syncthreads();  // the activation buffers are free for the results

  // ---- results through LDS in passes of MTP activation tiles: lane holds
  // C[m0 + 16 mt + 4 kg + e][n0 + 16 ns + ln]; each thread then writes 16-byte row chunks
  constexpr int PITCH = TR + 4;  // floats per LDS row (skewed)
  constexpr int PR = (2 * XBYTES / 4) / PITCH / 16 * 16;
  constexpr int MTP = PR / 16 >= MT ? MT : (PR / 16 >= 4 ? 4 : (PR / 16 >= 2 ? 2 : 1));
  static_assert(PR >= 16 && MT % MTP == 0, "whole passes");
  float* const s_t = reinterpret_cast<float*>(s_dyn);
  const bool split = ks > 1;
  const bool vec_n = p.n % 4 == 0;
  const bool vec_out = vec_n && p.o_stride % 4 == 0 && ((uintptr_t)p.out & 7) == 0;
  // two ranges with arrival words (N % 4 == 0): partials stored at device scope, and the
  // second range to finish a tile adds both (below) instead of a second kernel
  const bool fused = ks == 2 && arrivals != nullptr;
  const __amdgpu_buffer_rsrc_t rp =
      buffer_rsrc(part + ((int64_t)zr * p.m + m0) * p.n, (uint32_t)((int64_t)rows * p.n * 4));
#pragma unroll
  for (int mt0 = 0; mt0 < MT; mt0 += MTP) {
    if (mt0 > 0) __syncthreads();  // the previous pass has been read
#pragma unroll
    for (int mt = mt0; mt < mt0 + MTP; ++mt)
#pragma unroll
      for (int ns = 0; ns < NS; ++ns)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          s_t[(16 * (mt - mt0) + 4 * kg + e) * PITCH + wave * 16 * NS + 16 * ns + ln] = acc[mt][ns][e];
    __syncthreads();
    for (int q = threadIdx.x; q < 16 * MTP * (TR / 4); q += NTHR) {
      const int rl = q / (TR / 4), c4 = q - rl * (TR / 4);
      const int m = m0 + 16 * mt0 + rl, n = nb + 4 * c4;
      if (m >= p.m || n >= p.n) continue;
      const f32x4 v = *reinterpret_cast<const f32x4*>(&s_t[rl * PITCH + 4 * c4]);
      if (fused) {
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rp, ((m - m0) * p.n + n) * 4, 0,
                                               kDeviceScope);
      } else if (split) {
        float* const dst = part + ((int64_t)zr * p.m + m) * p.n + n;
        if (vec_n) {
          *reinterpret_cast<f32x4*>(dst) = v;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < p.n) dst[e] = v[e];
        }
      } else {
        T* const o = (T*)p.out + (int64_t)m * p.o_stride + n;
        if (vec_out) {
          const T h[4] = {(T)v[0], (T)v[1], (T)v[2], (T)v[3]};
          *reinterpret_cast<u32x2*>(o) = __builtin_bit_cast(u32x2, h);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < p.n) o[e] = (T)v[e];
        }
      }
    }
  }
  if (!fused) return;

  // Two ranges: the second to arrive at the tile reads both ranges' partials (device
  // scope: the other range's came from another CU, possibly another XCD) and writes
  // (0 + p0) + p1, the reduce kernel's sums in its order, whichever range arrives last
  __shared__ int s_last;
  wait_vm0();       // this thread's partials have reached the point of device coherence
  __syncthreads();  // every thread's, before the count moves
  if (threadIdx.x == 0) s_last = arrive_last(arrivals + (pair / ks) * m_blocks + (within >> 3), tag, ks) ? 1 : 0;
  __syncthreads();
  if (!s_last) return;
  const __amdgpu_buffer_rsrc_t r0 = buffer_rsrc(part + (int64_t)m0 * p.n, (uint32_t)((int64_t)rows * p.n * 4));
  const __amdgpu_buffer_rsrc_t r1 =
      buffer_rsrc(part + ((int64_t)p.m + m0) * p.n, (uint32_t)((int64_t)rows * p.n * 4));
  for (int q = threadIdx.x; q < BM * (TR / 4); q += NTHR) {
    const int rl = q / (TR / 4), c4 = q - rl * (TR / 4);
    const int m = m0 + rl, n = nb + 4 * c4;
    if (m >= p.m || n >= p.n) continue;
    const int off = (rl * p.n + n) * 4;
    const f32x4 p0 = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r0, off, 0, kDeviceScope));
    const f32x4 p1 = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r1, off, 0, kDeviceScope));
    f32x4 y;
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = (0.f + p0[e]) + p1[e];
    T* const o = (T*)p.out + (int64_t)m * p.o_stride + n;
    if (vec_out) {
      const T h[4] = {(T)y[0], (T)y[1], (T)y[2], (T)y[3]};
      *reinterpret_cast<u32x2*>(o) = __builtin_bit_cast(u32x2, h);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = (T)y[e];  // N % 4 == 0: the chunk is whole
    }
  }
}

// Skinny kernel (2 <= m <= 16, and up to m = 64 for 4096 x 4096, g == 128): bandwidth-
// bound shapes without a K split across workgroups. A workgroup owns 16*NS weight rows and KW waves; wave w takes the
// 128*ST keys [w*128*ST, (w+1)*128*ST) of those rows and of the 16*MT activation rows,
// P stages of 128 keys in flight (weights non-temporal). Per stage and weight tile: four
// MFMAs G = sum x (MAGIC + q), and per activation tile four MFMAs X = sum x against an
// all-ones operand; the fold acc += s G - s (MAGIC + z) X is exact for any zero point.
// The waves' partial sums meet in LDS and are added in wave order (deterministic).
//   - A stage is one quantisation group (g == 128), so a lane needs the scale and zero
//     point of its own weight row for ST consecutive groups: one load each for all its
//     stages, issued before the stream (scattered per-stage scale loads took the
//     address unit's cycles from the weight stream).
//   - Activations: instruction s of a stage reads rows 4 s .. 4 s + 3 of the tile, 256
//     contiguous bytes each (whole cache lines; the MFMA layout read directly from memory
//     -- 16 rows x 64 bytes per instruction at the rows' stride -- measured about twice as
//     slow on the activation side), and the wave writes the stage to its own LDS buffer
//     and reads it back in the MFMA A layout (rows padded by 16 bytes: no bank conflicts).
//     The buffer is private to the wave, whose LDS operations run in order: no barrier.
template <typename T, int MT, int NS>
struct SkinnyStage {
  u32x4 xa[MT][4];  // activation rows 4 s + kg of the tile, keys 8 (lane & 15) .. + 7 of the stage
  u32x4 w[NS];      // 32 nibbles: row 16 ns + (lane & 15), keys 32 kg .. + 31
};
constexpr int kSkinnyXRow = 256 + 16;  // LDS bytes of one staged activation row (128 keys + pad)

template <typename T, int MT, int NS, int ST, int P, int LB>
__global__ __launch_bounds__(LB) void w4a16_skinny_kernel(const W4Params p) {
  typedef W4Elem<T> E;
  typedef SkinnyStage<T, MT, NS> Stage;
  extern __shared__ __attribute__((aligned(16))) char s_dyn[];
  constexpr int NE = MT * NS * 4;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kw = blockDim.x >> 6;
  float* const s_red = (float*)s_dyn;  // [KW][MT * NS * 4][64]
  char* const s_xw = s_dyn + (size_t)kw * NE * 64 * 4 + (size_t)wave * MT * 16 * kSkinnyXRow;  // this wave's
  const int ln = lane & 15, kg = lane >> 4;
  const int n0 = blockIdx.x * 16 * NS;
  const int m0 = blockIdx.y * 16 * MT;
  const int rows = min(16 * MT, p.m - m0);
  const int k0 = wave * 128 * ST;
  const uint32_t magic = in_vgpr(E::kMagicPair);

  // scale and zero point of this lane's rows for the wave's ST groups (g == 128): ST
  // scales of esize bytes and ST int32 zero points, contiguous in each row
  const int esize = p.sdt == SS_DTYPE_F32 ? 4 : 2;
  const uint32_t f16_mask = p.sdt == SS_DTYPE_F16 ? ~0u : 0u, bf16_mask = p.sdt == SS_DTYPE_BF16 ? ~0u : 0u;
  const __amdgpu_buffer_rsrc_t rsc = buffer_rsrc(p.sc, (uint32_t)((int64_t)p.n * p.groups * esize));
  const __amdgpu_buffer_rsrc_t rzp = buffer_rsrc(p.qz, (uint32_t)((int64_t)p.n * p.groups * 4));
  // ST fp32 scales, or ST 16-bit scales from the dword holding the first (ST / 2 + 1
  // dwords cover them whether that one starts at a low or a high half). The same NSD
  // dwords are loaded for every scale dtype (the extra ones lie in the array or read as
  // zero past it): a load under a dtype condition made the compiler wait for it before
  // the stream's loads were issued, one memory round trip per call.
  constexpr int NSD = ST >= 2 ? ST : 1;
  uint32_t sdw[NS][NSD];
  int zv[NS][ST];
#pragma unroll
  for (int ns = 0; ns < NS; ++ns) {
    const int gi = min(n0 + 16 * ns + ln, p.n - 1) * p.groups + k0 / 128;
#pragma unroll
    for (int d = 0; d < NSD; ++d)
      sdw[ns][d] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rsc, (gi * esize & ~3) + 4 * d, 0, 0);
#pragma unroll
    for (int i = 0; i < ST; ++i) zv[ns][i] = __builtin_amdgcn_raw_buffer_load_b32(rzp, (gi + i) * 4, 0, 0);
  }
  // scale of stage i, tile ns: 16-bit scales start at the low half when gi is even
  auto stage_scale = [&](int ns, int i) {
    const int gi0 = min(n0 + 16 * ns + ln, p.n - 1) * p.groups + k0 / 128;
    uint32_t bits;
    if (esize == 4) {
      bits = sdw[ns][i];
    } else {
      const int h = (gi0 & 1) + i;  // 16-bit index from the first loaded dword
      bits = sdw[ns][h >> 1] >> (16 * (h & 1));
    }
    return decode_scale_masked(bits, f16_mask, bf16_mask);
  };

  // activation rows [m0, m0 + rows): a row past them reads as zero (its byte offset is at
  // least rows * x_stride * sizeof(T), past the descriptor's end as x_stride >= K)
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(
      (const T*)p.x + (int64_t)m0 * p.x_stride, (uint32_t)(((int64_t)(rows - 1) * p.x_stride + p.k) * sizeof(T)));
  int x_off[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int s = 0; s < 4; ++s)
      x_off[mt][s] = (int)(((int64_t)(16 * mt + 4 * s + kg) * p.x_stride + k0 + 8 * ln) * (int64_t)sizeof(T));
  // weight rows [n0, n0 + 16 NS) that exist; rows past N read as zero and are never stored
  const int live = min(16 * NS, p.n - n0);
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(p.qw + (int64_t)n0 * (p.k / 8), (uint32_t)live * (uint32_t)(p.k / 2));
  int w_off[NS];
#pragma unroll
  for (int ns = 0; ns < NS; ++ns) w_off[ns] = (16 * ns + ln) * (p.k / 2) + k0 / 2 + 16 * kg;

  auto issue = [&](int i, Stage& st) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int s = 0; s < 4; ++s)
        st.xa[mt][s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, x_off[mt][s], 256 * i, 0));
#pragma unroll
    for (int ns = 0; ns < NS; ++ns)
      st.w[ns] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, w_off[ns], 64 * i, kNonTemporal));
  };

  f32x4 acc[MT][NS];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) acc[mt][ns] = f32x4{0.f, 0.f, 0.f, 0.f};
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
  const uint32_t one2 = in_vgpr(E::kOnePair);
  const u32x4 ones = {one2, one2, one2, one2};

  auto compute = [&](Stage& st, int i) {
    u32x4 a[MT][4];
    f32x4 X[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      char* const tile = s_xw + mt * 16 * kSkinnyXRow;
#pragma unroll
      for (int s = 0; s < 4; ++s) store16(tile + (4 * s + kg) * kSkinnyXRow + 16 * ln, st.xa[mt][s]);
#pragma unroll
      for (int s = 0; s < 4; ++s) a[mt][s] = permute_x(load16(tile + ln * kSkinnyXRow + 64 * kg + 16 * s));
      X[mt] = Elem<T>::mfma(a[mt][0], ones, zero4);
#pragma unroll
      for (int s = 1; s < 4; ++s) X[mt] = Elem<T>::mfma(a[mt][s], ones, X[mt]);
    }
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) {
      f32x4 G[MT];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const u32x4 b = nibbles_to_operand(st.w[ns][s], magic);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) G[mt] = Elem<T>::mfma(a[mt][s], b, s == 0 ? zero4 : G[mt]);
      }
      const float sc = stage_scale(ns, i);
      const float szm = sc * (E::kMagic + (float)zv[ns][i]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[mt][ns][e] = fmaf(sc, G[mt][e], fmaf(-szm, X[mt][e], acc[mt][ns][e]));
    }
  };

  Stage ring[P];
#pragma unroll
  for (int u = 0; u < P; ++u) issue(u, ring[u]);
#pragma unroll
  for (int i = 0; i < ST; ++i) {
    compute(ring[i % P], i);
    if (i + P < ST) {
      __builtin_amdgcn_sched_barrier(0);
      issue(i + P, ring[i % P]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // the waves' K slices, added in wave order
  float* mine = s_red + (size_t)wave * NE * 64;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int ns = 0; ns < NS; ++ns)
#pragma unroll
      for (int e = 0; e < 4; ++e) mine[((mt * NS + ns) * 4 + e) * 64 + lane] = acc[mt][ns][e];
  __syncthreads();
  for (int t = threadIdx.x; t < NE * 64; t += blockDim.x) {
    float y = 0.f;
    for (int w2 = 0; w2 < kw; ++w2) y += s_red[(size_t)w2 * NE * 64 + t];
    const int idx = t >> 6, l = t & 63;
    const int e = idx & 3, ns = (idx >> 2) % NS, mt = (idx >> 2) / NS;
    const int m = m0 + 16 * mt + 4 * (l >> 4) + e;
    const int n = n0 + 16 * ns + (l & 15);
    if (m < p.m && n < p.n) ((T*)p.out)[(int64_t)m * p.o_stride + n] = (T)y;
  }
}

// out[m][n] = sum over ranges z (in order) of part[z][m][n]; VEC consecutive n per thread.
template <typename T, int VEC>
__global__ __launch_bounds__(256) void w4a16_splitk_reduce_kernel(const float* __restrict__ part, void* out, int m,
                                                                  int n, int splits, int64_t o_stride) {
  const int64_t per_row = n / VEC;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)m * per_row) return;
  const int r = (int)(idx / per_row);
  const int c = (int)(idx - (int64_t)r * per_row) * VEC;
  const int64_t plane = (int64_t)m * n;
  const float* src = part + (int64_t)r * n + c;
  float s[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) s[v] = 0.f;
  // eight ranges' loads in flight at a time, added in range order
  for (int z0 = 0; z0 < splits; z0 += 8) {
    float t[8][VEC];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int z = min(z0 + j, splits - 1);
      if (VEC == 4) {
        const f32x4 v4 = *reinterpret_cast<const f32x4*>(src + z * plane);
#pragma unroll
        for (int v = 0; v < VEC; ++v) t[j][v] = v4[v];
      } else {
#pragma unroll
        for (int v = 0; v < VEC; ++v) t[j][v] = src[z * plane + v];
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int v = 0; v < VEC; ++v) s[v] += z0 + j < splits ? t[j][v] : 0.f;
  }
  T* dst = (T*)out + (int64_t)r * o_stride + c;
#pragma unroll
  for (int v = 0; v < VEC; ++v) dst[v] = (T)s[v];
}

template <typename T>
__device__ __forceinline__ float elem_to_f32(T v) {
  return (float)v;
}

template <typename T>
__global__ __launch_bounds__(256) void w4a16_generic_kernel(const W4Params p) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)p.m * p.n) return;
  const int m = (int)(idx / p.n), n = (int)(idx - (int64_t)m * p.n);
  const T* xr = (const T*)p.x + (int64_t)m * p.x_stride;
  const uint32_t* wr = p.qw + (int64_t)n * (p.k >> 3);
  float acc = 0.f;
  for (int j = 0; j < (p.k >> 3); ++j) {
    const uint32_t w = wr[j];
    const int gi = (8 * j) / p.g;
    const int64_t si = (int64_t)n * p.groups + gi;
    const float s = load_scale(p.sc, si, p.sdt);
    const float z = (float)p.qz[si];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc = fmaf(elem_to_f32(xr[8 * j + i]), ((float)((w >> (4 * i)) & 15u) - z) * s, acc);
  }
  ((T*)p.out)[(int64_t)m * p.o_stride + n] = (T)acc;
}

// ---- host side -------------------------------------------------------------

// Batch-1 (decode) W4A16 GEMV, shaped for HBM bandwidth rather than MFMA tiles.
// A workgroup owns 16 weight rows; each of its waves owns one contiguous slice of
// K (128 IT keys). Eight consecutive lanes share a row and read 128 contiguous
// bytes of it (256 keys, one 16-byte load each), so a load instruction moves 8
// whole 128-byte lines (rows 0-7 or 8-15 of the workgroup), non-temporal: with
// 4 lanes per row (16 half lines per instruction) the same weights streamed 5-13 %
// slower. Every wave issues all its loads up front, so the whole matrix is
// requested at once. The activation rows
// are staged in LDS once per workgroup, permuted to the nibble order, with the
// sum of every 32 keys. Per 16-byte piece (32 keys of one row, one quantisation
// group as g % 32 == 0) a lane computes G = sum x (MAGIC + q) with v_dot2 and
// folds s * (G - (MAGIC + z) * X) into the sum of its row (two rows per lane); the
// eight lanes of a row add by DPP, the waves' slices add in LDS in wave order (no
// atomics: the result does not depend on timing).
//
// LDS: x [MR][K] permuted | chunk sums [K/32][MR] floats | slice partials [waves][16][MR] floats
// MR: activation rows held (the kernel is used with MR = 1). IT: 128-key iterations
// per wave (8: 1024-key slices for K <= 8192; 16: 2048-key slices for K <= 16384),
// so a workgroup has at most 8 waves.
template <typename T, int MR, int IT>
__global__ __launch_bounds__(512) void w4a16_gemv_kernel(const W4Params p) {
  typedef W4Elem<T> E;
  extern __shared__ __attribute__((aligned(16))) char s_dyn[];
  const int K = p.k;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  const int n0 = blockIdx.x * 16;
  // lane: row rl of each 8-row group, 32-key piece q8 of each 256 keys; load u
  // covers row group u & 1 and keys k0 + 256 (u >> 1) + 32 q8 .. + 31
  const int rl = lane >> 3, q8 = lane & 7;
  const int k0 = wave * 128 * IT;

  // Load order matters: the vector-memory counter retires loads in order, so the
  // activation pieces each thread stages are requested first, then the scales and
  // zero points, then this wave's weights (IT x 16 bytes per lane). The staging
  // below waits for the activations only, and iteration u of the dot products for
  // weight load u only, so the arithmetic overlaps the weight stream.
  // blockDim = 64 * K / (128 IT), so every thread stages exactly MR * IT / 4 pieces of
  // 8 keys.
  T* s_x = (T*)s_dyn;
  float* s_xs = (float*)(s_dyn + (size_t)MR * K * sizeof(T));
  float* s_part = s_xs + (size_t)(K / 32) * MR;
  u32x4 xin[MR * IT / 4];
#pragma unroll
  for (int e2 = 0; e2 < MR * IT / 4; ++e2) {
    const int e = threadIdx.x + e2 * blockDim.x;
    const int r = e / (K / 8), c8 = e - r * (K / 8);
    const u32x4 z = {0u, 0u, 0u, 0u};
    xin[e2] = r < p.m ? load16((const T*)p.x + (int64_t)r * p.x_stride + 8 * c8) : z;
  }
  const int esize = p.sdt == SS_DTYPE_F32 ? 4 : 2;
  const __amdgpu_buffer_rsrc_t rsc = buffer_rsrc(p.sc, (uint32_t)((int64_t)p.n * p.groups * esize));
  const __amdgpu_buffer_rsrc_t rzp = buffer_rsrc(p.qz, (uint32_t)((int64_t)p.n * p.groups * 4));
  uint32_t sb[IT];
  int zi[IT];
#pragma unroll
  for (int u = 0; u < IT; ++u) {
    const int row = n0 + 8 * (u & 1) + rl;
    const int64_t gi = (int64_t)(row < p.n ? row : 0) * p.groups + (k0 + 256 * (u >> 1) + 32 * q8) / p.g;
    sb[u] = scale_bits(rsc, gi, esize);
    zi[u] = __builtin_amdgcn_raw_buffer_load_b32(rzp, (int)(gi * 4), 0, 0);
  }
  // one descriptor over the workgroup's rows (rows past N read as zero)
  const int live_rows = min(16, p.n - n0);
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(p.qw + (int64_t)n0 * (K / 8), (uint32_t)live_rows * (uint32_t)(K / 2));
  const int vrow = rl * (K / 2) + k0 / 2 + 16 * q8;
  u32x4 wv[IT];
#pragma unroll
  for (int u = 0; u < IT; ++u)
    wv[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                          rw, vrow, (u & 1) * 4 * K + 128 * (u >> 1), kNonTemporal));

  // activations -> LDS (permuted to the nibble order), then per-32-key sums
#pragma unroll
  for (int e2 = 0; e2 < MR * IT / 4; ++e2) {
    const int e = threadIdx.x + e2 * blockDim.x;
    const int r = e / (K / 8), c8 = e - r * (K / 8);
    store16(s_x + (size_t)r * K + 8 * c8, permute_x(xin[e2]));
  }
  __syncthreads();
  for (int e = threadIdx.x; e < MR * (K / 32); e += blockDim.x) {
    const int r = e / (K / 32), c = e - r * (K / 32);
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x4 v = load16(s_x + (size_t)r * K + 32 * c + 8 * j);
#pragma unroll
      for (int h = 0; h < 4; ++h) sum += E::to_f32(v[h] & 0xFFFFu) + E::to_f32(v[h] >> 16);
    }
    s_xs[c * MR + r] = sum;
  }
  __syncthreads();

  // dot products, one 32-key piece per iteration, folded per quantisation group
  const uint32_t magic = in_vgpr(E::kMagicPair);
  float acc[2][MR];
#pragma unroll
  for (int g2 = 0; g2 < 2; ++g2)
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[g2][r] = 0.f;
#pragma unroll
  for (int u = 0; u < IT; ++u) {
    const int c = (k0 + 256 * (u >> 1)) / 32 + q8;
    u32x4 dq[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) dq[j] = nibbles_to_operand(wv[u][j], magic);
    const float zf = E::kMagic + (float)zi[u];
    const float sci = decode_scale(sb[u], p.sdt);
#pragma unroll
    for (int r = 0; r < MR; ++r) {
      float gsum = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x4 xv = load16(s_x + (size_t)r * K + 32 * c + 8 * j);
#pragma unroll
        for (int h = 0; h < 4; ++h) gsum = dot2_acc<T>(dq[j][h], xv[h], gsum);
      }
      acc[u & 1][r] += sci * (gsum - zf * s_xs[c * MR + r]);
      // finish this iteration's dot products here: left to itself the compiler
      // unpacks every iteration's weights as they land and defers all dot products
      // to the end, holding IT x 16 unpacked registers
      asm volatile("" : "+v"(acc[u & 1][r]));
    }
  }

  // the eight lanes of a row, then the waves' slices in order
#pragma unroll
  for (int g2 = 0; g2 < 2; ++g2)
#pragma unroll
    for (int r = 0; r < MR; ++r) {
      float v = acc[g2][r];
      v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
      v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
      v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true));
      if (q8 == 0) s_part[(wave * 16 + 8 * g2 + rl) * MR + r] = v;
    }
  __syncthreads();
  if (threadIdx.x < 16 * MR) {
    const int rr = threadIdx.x / MR, r = threadIdx.x - rr * MR;
    float y = 0.f;
    for (int w = 0; w < nw; ++w) y += s_part[(w * 16 + rr) * MR + r];
    if (r < p.m && n0 + rr < p.n) ((T*)p.out)[(int64_t)r * p.o_stride + n0 + rr] = (T)y;
  }
}

// Narrow kernel (1 <= m <= 4, g == 128): the small-batch GEMV with its dot products on
// MFMA 16x16x32 instead of v_dot2, which leaves the VALU only the nibble unpack (seven
// instructions per 32-bit word) and two FMAs per activation row and load.
//
// A workgroup owns 4 J weight rows; its waves split K into slices of W 512-key windows.
// One weight load instruction moves 4 rows x 256 contiguous bytes (one window of each):
// MFMA B column c is row c >> 2, piece c & 3 (128 keys = one group) of the window, and
// the four lanes of a column (k-blocks kg) hold 32 consecutive keys of it, one 32-bit
// word per MFMA. A row a holds activation row a & 3 over piece a >> 2. Product entry
// (a, c) is a dot product of the same keys only where the pieces agree (a >> 2 == c & 3):
// lane 16 (c & 3) + c holds those entries of column c, element i = activation row i, as
// G = sum over the group of x (MAGIC + q). The same A against an all-ones B gives X =
// sum x of (row, piece) in the same lanes and elements, so the fold s G - s (MAGIC + z) X
// applies to the MFMA outputs directly. The other entries are computed and dropped (the
// matrix unit has the cycles: 4 MFMAs per 2048 weights).
//
// Each wave stages its own activation slice in its own LDS rows (permuted to the nibble
// order; its LDS operations run in order, so no barrier), the weights stream straight
// into registers (all J W loads issued up front, consumed in order as they land), and
// the waves' slices and the four pieces of each row add in LDS in a fixed order.
// SD: the scale dtype.
//
// LDS: x [waves][MR][512 W] permuted | partials [waves][4 J rows][MR][4 pieces] floats |
//      (scale, MAGIC + zero) [waves][4 J rows][4 W groups] float pairs
template <int SD>
__device__ __forceinline__ float narrow_scale(uint32_t bits) {
  if constexpr (SD == SS_DTYPE_F16) return (float)__builtin_bit_cast(f16_t, (uint16_t)(bits & 0xFFFFu));
  if constexpr (SD == SS_DTYPE_BF16) return __builtin_bit_cast(float, bits << 16);
  return __builtin_bit_cast(float, bits);
}

template <typename T, int MR, int J, int W, int SD>
__global__ __launch_bounds__(512) void w4a16_narrow_kernel(const W4Params p) {
  typedef W4Elem<T> E;
  extern __shared__ __attribute__((aligned(16))) char s_dyn[];
  constexpr int SL = 512 * W;  // keys of a wave's slice
  constexpr int IT = J * W;    // weight loads per lane
  const int K = p.k;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  const int n0 = blockIdx.x * 4 * J;
  const int c = lane & 15, kg = lane >> 4;
  const int cr = c >> 2, cp = c & 3;  // column c: row cr of a four-row load, piece cp of the window
  const int k0 = wave * SL;
  T* const s_xw = (T*)s_dyn + (size_t)wave * MR * SL;
  float* const s_part = (float*)(s_dyn + (size_t)nw * MR * SL * sizeof(T));
  // the wave's (scale, MAGIC + zero) pairs [4 J rows][4 W groups], after the partials
  float2* const s_sz = (float2*)(s_part + (size_t)nw * 4 * J * MR * 4) + (size_t)wave * 16 * J * W;
  // Loads in the order they are consumed (the vector-memory counter retires in order):
  // the activation slice, the scales and zero points, then the weights.
  // Activation rows at or past m read as zero: their offsets start past the
  // descriptor's end since x_stride >= K.
  const __amdgpu_buffer_rsrc_t rx =
      buffer_rsrc(p.x, (uint32_t)(((int64_t)(p.m - 1) * p.x_stride + K) * sizeof(T)));
  u32x4 xin[MR * W];
#pragma unroll
  for (int e2 = 0; e2 < MR * W; ++e2) {
    const int q = lane + 64 * e2;
    const int r = q / (64 * W), c8 = q - r * (64 * W);
    xin[e2] = __builtin_bit_cast(
        u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)((r * p.x_stride + k0 + 8 * c8) * sizeof(T)), 0, 0));
  }
  // The (scale, zero) block of the wave's rows and groups: lane (row lr, part lh) reads
  // IT / 4 consecutive groups of its row (rows past N read as zero, past the
  // descriptors' ends); decoded once into LDS below.
  static_assert(IT == 8 || IT == 16, "two or four groups per lane in the scale block");
  static_assert(SD >= 0, "a fixed scale dtype");
  constexpr int esize = SD == SS_DTYPE_F32 ? 4 : 2;
  const __amdgpu_buffer_rsrc_t rsc = buffer_rsrc(p.sc, (uint32_t)((int64_t)p.n * p.groups * esize));
  const __amdgpu_buffer_rsrc_t rzp = buffer_rsrc(p.qz, (uint32_t)((int64_t)p.n * p.groups * 4));
  constexpr int LPR = 16 / J;  // lanes per row
  const int lr = lane / LPR, lh = lane - lr * LPR;
  const int gq = (n0 + lr) * p.groups + k0 / 128 + lh * (IT / 4);
  u32x4 zq = {0u, 0u, 0u, 0u}, sq = {0u, 0u, 0u, 0u};
  if constexpr (IT == 16) {
    zq = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rzp, gq * 4, 0, 0));
    if constexpr (esize == 4) {
      sq = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsc, gq * 4, 0, 0));
    } else {
      const u32x2 t = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rsc, gq * 2, 0, 0));
      sq = u32x4{t[0] & 0xFFFFu, t[0] >> 16, t[1] & 0xFFFFu, t[1] >> 16};
    }
  } else {
    const u32x2 z2 = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rzp, gq * 4, 0, 0));
    zq = u32x4{z2[0], z2[1], 0u, 0u};
    if constexpr (esize == 4) {
      const u32x2 t = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rsc, gq * 4, 0, 0));
      sq = u32x4{t[0], t[1], 0u, 0u};
    } else {
      const uint32_t t = __builtin_amdgcn_raw_buffer_load_b32(rsc, gq * 2, 0, 0);
      sq = u32x4{t & 0xFFFFu, t >> 16, 0u, 0u};
    }
  }
  // one descriptor over the workgroup's rows (rows past N read as zero)
  const int live_rows = min(4 * J, p.n - n0);
  const __amdgpu_buffer_rsrc_t rw =
      buffer_rsrc(p.qw + (int64_t)n0 * (K / 8), (uint32_t)live_rows * (uint32_t)(K / 2));
  const int vrow = cr * (K / 2) + k0 / 2 + 64 * cp + 16 * kg;
  u32x4 wv[IT];
#pragma unroll
  for (int u = 0; u < IT; ++u) {
    const int w = u / J, j = u - w * J;
    wv[u] = __builtin_bit_cast(u32x4,
                               __builtin_amdgcn_raw_buffer_load_b128(rw, vrow, j * 2 * K + 256 * w, kNonTemporal));
  }

  // the wave's activation slice -> its LDS rows, permuted to the nibble order
#pragma unroll
  for (int e2 = 0; e2 < MR * W; ++e2) {
    const int q = lane + 64 * e2;
    const int r = q / (64 * W), c8 = q - r * (64 * W);
    store16(s_xw + r * SL + 8 * c8, permute_x(xin[e2]));
  }
#pragma unroll
  for (int e = 0; e < IT / 4; ++e)
    s_sz[lr * 4 * W + lh * (IT / 4) + e] = make_float2(narrow_scale<SD>(sq[e]), E::kMagic + (float)(int)zq[e]);
  __builtin_amdgcn_wave_barrier();

  const uint32_t magic = in_vgpr(E::kMagicPair);
  const uint32_t one2 = in_vgpr(E::kOnePair);
  const u32x4 ones = {one2, one2, one2, one2};
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
  // A row c of this lane: activation row c & 3 (a duplicate where m has fewer rows)
  const int xr = MR == 1 ? 0 : (MR == 2 ? (cp & 1) : cp);
  f32x4 tot[J];
#pragma unroll
  for (int j = 0; j < J; ++j) tot[j] = zero4;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    u32x4 a[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) a[s] = load16(s_xw + xr * SL + 512 * w + 128 * cr + 32 * kg + 8 * s);
    f32x4 X = Elem<T>::mfma(a[0], ones, zero4);
#pragma unroll
    for (int s = 1; s < 4; ++s) X = Elem<T>::mfma(a[s], ones, X);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int u = w * J + j;
      f32x4 G = Elem<T>::mfma(a[0], nibbles_to_operand(wv[u][0], magic), zero4);
#pragma unroll
      for (int s = 1; s < 4; ++s) G = Elem<T>::mfma(a[s], nibbles_to_operand(wv[u][s], magic), G);
      const float2 sz = s_sz[(4 * j + cr) * 4 * W + 4 * w + cp];
#pragma unroll
      for (int i = 0; i < MR; ++i) tot[j][i] = fmaf(sz.x, fmaf(-sz.y, X[i], G[i]), tot[j][i]);
    }
  }

  // lanes with kg == cp hold row 4 j + cr, piece cp; add pieces and waves in order
  if (kg == cp) {
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int i = 0; i < MR; ++i) s_part[((wave * 4 * J + 4 * j + cr) * MR + i) * 4 + cp] = tot[j][i];
  }
  __syncthreads();
  if (threadIdx.x < 4 * J * MR) {
    const int rr = threadIdx.x / MR, i = threadIdx.x - rr * MR;
    float y = 0.f;
    for (int w2 = 0; w2 < nw; ++w2) {
      const float* q = s_part + ((w2 * 4 * J + rr) * MR + i) * 4;
      y += (q[0] + q[1]) + (q[2] + q[3]);
    }
    if (i < p.m && n0 + rr < p.n) ((T*)p.out)[(int64_t)i * p.o_stride + n0 + rr] = (T)y;
  }
}

struct W4Plan {
  bool fast;
  bool wide;
  bool xlds;
  int narrow;  // activation rows of the narrow kernel (1, 2 or 4), 0: not used
  int gemv;  // 1: the batch-1 GEMV kernel
  bool tile;  // the tiled kernel (activations shared through LDS)
  bool skinny;  // the skinny kernel (m <= 64, K split over the waves of one workgroup)
  bool widek;   // the wide kernel (m > 64, weights dequantised once per wave)
  int st;       // skinny: 128-key stages per wave
  int mt, ns, bit, kw, pf;
  int m_blocks, n_tiles;
  int ks, kchunk;  // tiled kernel: K ranges and 128-key stages per range
  size_t lds;
};

// Tiled kernel for m >= 2 when g % 128 == 0 and K is a whole number of PF-stage
// rounds. Shapes (activation tiles MT, weight tiles NS per wave, prefetch depth PF)
// by m: two stages of weights in flight per wave everywhere (at m = 32 against eight:
// 4096 x 6144 12.2 vs 14.2 us, 14336 x 4096 17.0 vs 19.5 us; at m = 48 / 64 against
// four: 16.5 vs 17.3 us, 4096 x 4096 15.9 vs 16.5 us at m = 64; a shallower ring also
// gives the K split more rounds to divide); m > 32 takes 64 x 32 wave tiles (at m = 128
// / 256 against 64 x 64: 4096 x 6144 25.5 / 30.0 vs 28.5 / 36.5 us, 4096 x 14336 31.5 /
// 50.0 vs 37.4 / 51.6 us, 4096 x 28672 52.4 / 96.3 vs 54.8 / 100.4 us). The K
// split aims at one workgroup
// per CU for m <= 64 and two for m > 64 (the nearest whole count of ranges: 224
// weight tiles at m <= 64 stay unsplit), in ranges of equal length (the split count
// divides the rounds of PF stages), with the workgroup's scale table within
// kTileTableMax bytes of LDS; the partials take ks * m * n floats of workspace.
// Measured over the Llama-3-8B linears (kernel + reduce), e.g. 4096 x 6144 at
// m = 64: 19.9 us for 4 ranges against 22.9 us for 8 and 22.7 us for 3 uneven
// ones; 4096 x 28672 at m = 64: 39.9 us unsplit against 46.6 us for 3 ranges;
// 14336 x 4096 at m = 256: 56.4 us for 8 ranges against 66.0 us for 4; 4096 x 28672
// (224 tiles) at m = 32 / 64: 23.2 / 33.1 us unsplit against 26.8 / 34.3 us for two
// ranges finished in-kernel; at m = 192 rounding to the nearest count rather than up
// takes 4096 x 6144 from 8 ranges to 4 (37.1 -> 35.8 us) and 4096 x 14336 from 4 to 2
// (52.9 -> 51.2 us). The
// table cap keeps two workgroups per CU: with the 35 KB activation stages of
// m > 32, a 64 KB table left room for one (a 4096 x 28672 linear at m = 256 took
// 233 us instead of 2 x 67 us).
constexpr int kTileTableMax = 40 * 1024;

size_t tile_table_bytes(int ns, int kchunk, int g) {
  const int gr = (kchunk * 128 + g - 1) / g + 1;  // groups a range can touch
  return (size_t)64 * ns * (gr + 1) * 8;
}

bool plan_tile(W4Plan& pl, int64_t m, int64_t n, int64_t k, int g) {
  if (!pl.wide || m < 2) return false;
  // m <= 16 is weight-bandwidth bound and the untiled kernel shares activations
  // well enough there; for K < 8192 it measured faster (no reduction launch) up to
  // N = 14336 (11.5 vs 12.8 us at 4096 x 6144), the tiled one from N = 28672 (26.9 vs
  // 30.9 us at 4096 x 28672, the stacked gate/up projection)
  if (m <= 16 && k < 8192 && n < 24576) return false;
  int mt, ns, pf;
  if (m <= 16)
    mt = 1, ns = 2, pf = 2;
  else if (m <= 32)
    mt = 2, ns = 2, pf = 2;
  else
    mt = 4, ns = 2, pf = 2;
  // small grids (64-row blocks x 128-row weight tiles at most half the CUs, K <= 8192):
  // 32-row activation tiles, twice the workgroups before any K split (m = 64: 4096 x
  // 6144 14.6 vs 17.8 us, 4096 x 4096 12.7 vs 15.8, 4096 x 14336 20.4 vs 22.4; m = 256:
  // 4096 x 4096 21.6 vs 26.9 us); with larger K (14336 x 4096) or grids they are slower
  const bool small_grid =
      mt == 4 && k <= 8192 && ((n + 127) / 128) * ((m + 63) / 64) <= ss_host::device_cu_count() / 2;
  if (small_grid) mt = 2;
  const int64_t iters = k / 128;
  if (iters % pf) return false;
  const int64_t n_tiles = (n + 64 * ns - 1) / (64 * ns);
  const int64_t m_blocks = (m + 16 * mt - 1) / (16 * mt);
  if (n_tiles > 65535 || m_blocks > 65535) return false;
  // one workgroup per CU at m <= 64 and on small grids, two otherwise (m = 128: 4096 x
  // 4096 15.7 vs 18.1 us, 4096 x 6144 19.7 vs 21.2 with one; 14336 x 4096 at m = 256
  // 52.5 with two against 61.1 with one)
  const int64_t target = (m <= 64 || small_grid ? 1LL : 2LL) * ss_host::device_cu_count();
  const int64_t tiles = n_tiles * m_blocks;
  const int64_t rounds = iters / pf;
  int64_t ks = (target + tiles / 2) / tiles;
  ks = ks < 1 ? 1 : (ks > rounds ? rounds : ks);
  while (ks > 1 && rounds % ks) --ks;  // equal ranges
  if (ks > 65535) return false;
  // more ranges while a range's scale table is too large; the ranges stay balanced
  int64_t per = (rounds + ks - 1) / ks;
  while (per > 1 && tile_table_bytes(ns, (int)(per * pf), g) > (size_t)kTileTableMax) {
    ++ks;
    per = (rounds + ks - 1) / ks;
  }
  if (tile_table_bytes(ns, (int)(per * pf), g) > (size_t)kTileTableMax) return false;
  pl.tile = true;
  pl.mt = mt, pl.ns = ns, pl.pf = pf;
  pl.n_tiles = (int)n_tiles;
  pl.m_blocks = (int)m_blocks;
  pl.kchunk = (int)(per * pf);
  pl.ks = (int)((rounds + per - 1) / per);
  if (pl.ks > 65535) return false;
  pl.lds = tile_table_bytes(ns, pl.kchunk, g);
  // the partials are addressed by 32-bit offsets, with kOutOfRange past all of them
  if (pl.ks > 1 && (int64_t)pl.ks * m * n * 4 >= (int64_t)kOutOfRange) return false;
  return true;
}

// Skinny kernel for 1 <= m <= 64 with g % 128 == 0: the K split stays inside one
// workgroup (K = KW waves x 128 ST keys, KW <= 16), so no partials leave it. Activation
// tiles MT = ceil(m / 16) (at most 4); NS = 2 weight tiles per wave when that still
// leaves >= 2048 waves (halves the activation reads), else 1.
constexpr size_t kSkinnyLdsMax = 128 * 1024;

bool plan_skinny(W4Plan& pl, int64_t m, int64_t n, int64_t k, int g) {
  if (!pl.wide || m < 2 || m > 64 || g != 128) return false;
  // 16 < m <= 64 only for the 4096 x 4096 class (one 16-row activation tile per
  // workgroup row, the weights re-read per tile from the L2 / MALL): o at m = 17 / 32 / 48
  // / 64 7.6 / 7.8 / 11.5 / 11.6 us against 9.9 / 11.2 / 12.0 / 12.7 on the tiled
  // kernel; wider or deeper linears lose (gate at m = 64 43.6 against 20.0, down 59.2
  // against 24.3)
  if (m > 16 && (n > 4096 || k > 4096)) return false;
  // the widest linears take the tiled kernel (the stacked gate/up projection, 4096 x
  // 28672, 224 weight tiles, unsplit: 22.2 against 24.0 us at m = 16, 22.0 against 22.7
  // at m = 8; for narrower N the skinny kernel stays well ahead)
  if (n >= 24576 && k < 8192) return false;
  const int64_t q = k / 128;
  int st = 0;
  for (int c : {4, 8, 2, 1})
    if (q % c == 0 && q / c <= 16) {
      st = c;
      break;
    }
  if (!st) return false;
  const int mt = 1;
  int kw = (int)(q / st);
  const int64_t m_blocks = (m + 16 * mt - 1) / (16 * mt);
  // four weight tiles per wave: each activation fragment serves 64 weight rows, so the
  // activation reads (L2) match the weight bytes; needs the 256 registers of a
  // workgroup of at most 8 waves (ST 4 or 8)
  // the fewest weight tiles per wave that keep the grid within one workgroup per CU:
  // every workgroup stages all of its activation rows' K, so fewer, wider workgroups
  // read fewer activation bytes (four tiles need at most 8 waves and 4 or 8 stages)
  const int64_t cus = ss_host::device_cu_count();
  int ns = 4;
  for (int c : {1, 2})
    if ((n + 16 * c - 1) / (16 * c) * m_blocks <= cus) {
      ns = c;
      break;
    }
  if (ns == 4 && (kw > 8 || st != 4)) ns = 2;  // four tiles: 256 registers (<= 8 waves), 4 stages
  if (ns == 2 && st > 4) ns = 1;                 // two tiles of 8 stages exceed 128 registers
  const size_t lds = (size_t)kw * mt * ns * 4 * 64 * 4 + (size_t)kw * mt * 16 * kSkinnyXRow;
  if (lds > kSkinnyLdsMax) return false;
  const int64_t n_tiles = (n + 16 * ns - 1) / (16 * ns);
  if (n_tiles > 0x7fffffff) return false;
  // activation fragments are addressed by 32-bit byte offsets within a 16*MT-row block
  pl.skinny = true;
  pl.mt = mt, pl.ns = ns, pl.st = st, pl.kw = kw;
  pl.n_tiles = (int)n_tiles;
  pl.m_blocks = (int)m_blocks;
  pl.lds = lds;
  return true;
}

// Split-K workspace of the tiled kernel: the fp32 partials [ranges][m][n], then (256-byte
// aligned) one 64-bit arrival word per output tile (weight tile x activation block).
// The wide kernel's: the partials alone.
int64_t tile_part_bytes(const W4Plan& pl, int64_t m, int64_t n) { return ((int64_t)pl.ks * m * n * 4 + 255) / 256 * 256; }
int64_t tile_workspace_bytes(const W4Plan& pl, int64_t m, int64_t n) {
  if (pl.widek) return pl.ks > 1 ? tile_part_bytes(pl, m, n) + (int64_t)pl.n_tiles * pl.m_blocks * 8 : 0;
  return pl.tile && pl.ks > 1 ? tile_part_bytes(pl, m, n) + (int64_t)pl.n_tiles * pl.m_blocks * 8 : 0;
}

// Wide kernel for m > 64 with g == 128: 128 x 256 workgroup tiles, K split over
// workgroups so that the grid holds about one workgroup per CU (the kernel's eight waves
// and its LDS allow one per CU), in ranges of equal length of at least 12 stages. (A
// 64 x 256 form for 16 < m <= 64 measured no faster than the tiled kernel: 4096 x 28672
// at m = 64 37.1 against 35.4 us.)
constexpr size_t kWideXLds = (size_t)2 * kWideMT * 16 * 256;  // two activation stages
constexpr size_t kWideLdsMax = 160 * 1024 - 256;  // the CU's LDS less the kernel's static bytes
size_t wide_lds_bytes(int ns, int kchunk) { return kWideXLds + (size_t)16 * ns * kWideWV * kchunk * 8; }

bool plan_wide(W4Plan& pl, int64_t m, int64_t n, int64_t k, int g) {
  if (!pl.wide || m <= 64 || g != 128) return false;
  static const int enabled = [] {
    const char* e = getenv("SLIPSTREAM_W4A16_WIDE");
    return e ? atoi(e) : 1;
  }();
  if (!enabled) return false;
  const int64_t stages = k / 128;
  if (stages % kWidePF) return false;  // ranges of whole PF-stage rounds
  const int64_t m_blocks = (m + 16 * kWideMT - 1) / (16 * kWideMT);
  // 256 weight rows per workgroup (two 16-row tiles a wave), or 128 (one) where 256-row
  // tiles would leave the grid under three quarters of the CUs before any K split (C5 at
  // m = 256: 4096 x 14336 unsplit on 128-row tiles 51.1 us, in two ranges on 256-row
  // tiles 53.6 us; the stacked 4096 x 28672 stays on 256-row tiles, unsplit, 78.5 us)
  int ns = kWideNS;
  if ((n + 16 * ns * kWideWV - 1) / (16 * ns * kWideWV) * m_blocks * 4 < 3 * ss_host::device_cu_count()) ns = 1;
  const int64_t n_tiles = (n + 16 * ns * kWideWV - 1) / (16 * ns * kWideWV);
  if (n_tiles > 65535 || m_blocks > 65535) return false;
  const int64_t tiles = n_tiles * m_blocks;
  const int64_t target = ss_host::device_cu_count();
  int64_t ks = (target + tiles / 2) / tiles;
  const int64_t rounds = stages / kWidePF;
  ks = ks < 1 ? 1 : (ks > rounds ? rounds : ks);
  int64_t per = (rounds + ks - 1) / ks * kWidePF;  // stages per range
  while (per > kWidePF && wide_lds_bytes(ns, (int)per) > kWideLdsMax) per -= kWidePF;  // the table fits
  if (wide_lds_bytes(ns, (int)per) > kWideLdsMax) return false;
  ks = (stages + per - 1) / per;
  per = (rounds + ks - 1) / ks * kWidePF;  // balanced again
  // short ranges leave the per-workgroup set-up and result traffic uncovered: below 16
  // stages the tiled kernel is faster (C5 at m = 256: 4096 x 6144 in 3 ranges of 12, 12
  // and 8 stages 43.8 against 32.1 us, in 4 ranges of 8 stages 36.6 against 31.8 us;
  // 4096 x 4096 in 8 ranges of 4 stages 32.3 against 22.0 us)
  if (per < 16) return false;
  ks = (stages + per - 1) / per;
  if (ks > 65535) return false;
  pl.widek = true;
  pl.mt = kWideMT, pl.ns = ns;
  pl.n_tiles = (int)n_tiles;
  pl.m_blocks = (int)m_blocks;
  pl.ks = (int)ks;
  pl.kchunk = (int)per;
  pl.lds = wide_lds_bytes(ns, (int)per);
  return true;
}

constexpr size_t kLdsBudget = 64 * 1024;  // LDS bytes per workgroup

W4Plan plan_w4a16(int64_t m, int64_t n, int64_t k, int g, bool act16, bool allow_tile = true) {
  W4Plan pl = {};
  pl.fast = act16 && k % 128 == 0 && g % 32 == 0 && k > 0 && n * k / 2 < ((int64_t)1 << 31);
  pl.wide = g % 128 == 0;
  if (!pl.fast) return pl;
  // batch 1: the bandwidth GEMV when K splits into at most 8 wave slices of 1024
  // keys (K <= 8192) or 2048 keys (K <= 16384) and the staged activation row fits
  // the LDS budget. (A second activation row makes the compiler hoist every
  // activation read and spill: m >= 2 takes the MFMA kernel.)
  const int gemv_slice = k <= 8192 ? 1024 : 2048;
  if (m <= 4 && g == 128 && k % gemv_slice == 0 && k <= 16384) {
    const int mr = m == 1 ? 1 : (m == 2 ? 2 : 4);
    const int64_t waves = k / gemv_slice;
    pl.narrow = mr;
    // x slices | partials | (scale, zero) pairs of 16 rows x slice / 128 groups
    pl.lds = (size_t)waves * mr * gemv_slice * 2 + (size_t)waves * 16 * mr * 4 * 4 + (size_t)waves * 16 * (gemv_slice / 128) * 8;
    pl.n_tiles = (int)((n + 15) / 16);
    return pl;
  }
  if (m == 1 && k % gemv_slice == 0 && k <= 16384) {
    const int mr = 1;
    const size_t lds = (size_t)mr * k * 2 + (size_t)(k / 32) * mr * 4 + (size_t)(k / gemv_slice) * 16 * mr * 4;
    if (lds <= kLdsBudget) {
      pl.gemv = mr;
      pl.lds = lds;
      pl.n_tiles = (int)((n + 15) / 16);
      return pl;
    }
  }
  if (plan_skinny(pl, m, n, k, g)) return pl;
  if (allow_tile && plan_wide(pl, m, n, k, g)) return pl;
  pl.widek = false;
  if (allow_tile && plan_tile(pl, m, n, k, g)) return pl;
  pl.tile = false;
  const size_t unit = pl.wide ? 128 : 32;
  const int64_t groups = k / g;
  const int iters = (int)(k / 128);
  const int64_t want = 8LL * ss_host::device_cu_count();  // waves in flight to cover HBM latency
  // x staged in LDS when one 16-row tile of it fits beside the scale table
  const int64_t rows1 = m < 16 ? m : 16;
  const size_t x1 = (size_t)rows1 * (k + 8) * 2 + (size_t)(k / unit) * 16 * 4;
  const size_t sz1 = (size_t)16 * (2 * groups + 2) * 4;
  if (m <= 16 && x1 + sz1 <= kLdsBudget) {
    pl.mt = 1, pl.ns = 1, pl.bit = 4, pl.xlds = true;
  } else if (m <= 16) {
    // 64 weight rows share each activation fragment, unless that leaves more than
    // half the CUs idle: then 32 (twice the activation reads, twice the workgroups;
    // measured faster for N = 4096 and 6144, slower for 14336)
    const int64_t cus = ss_host::device_cu_count();
    if ((n + 63) / 64 >= cus / 2)
      pl.mt = 1, pl.ns = 4, pl.bit = 2;
    else
      pl.mt = 1, pl.ns = 2, pl.bit = 2;
  } else if (m <= 32) {
    pl.mt = 2, pl.ns = 2, pl.bit = 2;
  } else {
    pl.mt = 4, pl.ns = 2, pl.bit = 1;
  }
  pl.m_blocks = (int)((m + 16 * pl.mt - 1) / (16 * pl.mt));
  pl.n_tiles = (int)((n + 16 * pl.ns - 1) / (16 * pl.ns));
  // K slices per workgroup, with at least two 128-key iterations per slice
  const int64_t wgs = (int64_t)pl.m_blocks * pl.n_tiles;
  pl.kw = wgs * 4 >= want ? 4 : kMaxKW;
  while (pl.kw > 1 && iters < 2 * pl.kw) pl.kw >>= 1;
  const size_t red = (size_t)(pl.kw - 1) * pl.mt * pl.ns * 64 * 16;
  const size_t xb = pl.xlds ? x1 : 0;
  const size_t szb = (size_t)16 * pl.ns * (2 * groups + 2) * 4;
  pl.lds = xb + szb > red ? xb + szb : red;  // the reduction reuses the tables' bytes
  if (pl.lds > kLdsBudget) pl.fast = false;  // scale table too large: scalar kernel
  return pl;
}

template <typename T, int MT, int NS, int BIT, bool X>
int launch_w4a16_x(const W4Params& p, const W4Plan& pl, hipStream_t stream) {
  dim3 grid((unsigned)pl.n_tiles, (unsigned)pl.m_blocks);
  dim3 block(64 * pl.kw);
  if (pl.wide)
    hipLaunchKernelGGL((w4a16_kernel<T, MT, NS, BIT, true, X>), grid, block, pl.lds, stream, p);
  else
    hipLaunchKernelGGL((w4a16_kernel<T, MT, NS, BIT, false, X>), grid, block, pl.lds, stream, p);
  return ss_host::launch_status("w4a16 gemm");
}

// Tag of a split call's arrival words: a process-wide count, so that words left by earlier
// calls (or never written) do not match.
unsigned long long next_arrival_tag() {
  static std::atomic<unsigned long long> count{0};
  unsigned long long t = 0;
  while (t == 0) t = (++count & ((1ull << 56) - 1)) << 8;
  return t;
}

// NS weight tiles per wave, WV waves: the plan's 64 * pl.ns rows per workgroup are
// 16 * NS * WV
template <typename T, int MT, int NS, int PF, int WV>
int launch_w4a16_tile(const W4Params& p, const W4Plan& pl, float* part, hipStream_t stream) {
  if (16 * NS * WV != 64 * pl.ns) {
    ss_host::set_error("w4a16 gemm: tiled plan of %d rows per workgroup, kernel of %d", 64 * pl.ns, 16 * NS * WV);
    return SS_ERR_UNSUPPORTED;
  }
  if (pl.kchunk % PF != 0) {  // the loop runs whole rounds of PF stages
    ss_host::set_error("w4a16 gemm: K range of %d stages for a %d-stage prefetch ring", pl.kchunk, PF);
    return SS_ERR_UNSUPPORTED;
  }
  static bool attr_set = false;  // per instantiation; the attribute is process-wide
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)w4a16_tile_kernel<T, MT, NS, PF, WV>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, kTileTableMax) != hipSuccess) {
      ss_host::set_error("w4a16 gemm: cannot reserve %d bytes of LDS", kTileTableMax);
      return SS_ERR_UNSUPPORTED;
    }
    attr_set = true;
  }
  const int64_t pairs = (int64_t)pl.ks * pl.n_tiles;
  const int64_t grid = (pairs + 7) / 8 * 8 * pl.m_blocks;
  if (grid > 0x7fffffff) {
    ss_host::set_error("w4a16 gemm: %lld tiled workgroups", (long long)grid);
    return SS_ERR_UNSUPPORTED;
  }
  // Two ranges (and whole 16-byte row chunks, N % 4 == 0): the last range of each tile
  // adds the other range's partials to its own itself (C5 gate and gate_up at m = 32 and
  // 64: 7-9 % faster than a second kernel; at m = 256 gate 51.4 against 54.8 us, gate_up
  // 99.3 against 101.2). With more ranges that last workgroup's gather outlasts a reduce
  // kernel spread over the whole GPU (o at m = 64, 8 ranges: 21.4 against 16.4 us).
  const bool fused = pl.ks == 2 && p.n % 4 == 0;
  unsigned long long* const arrivals = fused ? (unsigned long long*)((char*)part + tile_part_bytes(pl, p.m, p.n)) : nullptr;
  const unsigned long long tag = fused ? next_arrival_tag() : 0ull;
  hipLaunchKernelGGL((w4a16_tile_kernel<T, MT, NS, PF, WV>), dim3((unsigned)grid), dim3(64 * WV), pl.lds, stream, p,
                     part, arrivals, tag, pl.kchunk, pl.ks, pl.n_tiles, pl.m_blocks);
  int st = ss_host::launch_status("w4a16 gemm (tiled)");
  if (st != SS_OK || pl.ks == 1 || fused) return st;
  const bool vec = p.n % 4 == 0;
  const int64_t threads = (int64_t)p.m * (vec ? p.n / 4 : p.n);
  const unsigned blocks = (unsigned)((threads + 255) / 256);
  if (vec)
    hipLaunchKernelGGL((w4a16_splitk_reduce_kernel<T, 4>), dim3(blocks), dim3(256), 0, stream, part, p.out, p.m, p.n,
                       pl.ks, p.o_stride);
  else
    hipLaunchKernelGGL((w4a16_splitk_reduce_kernel<T, 1>), dim3(blocks), dim3(256), 0, stream, part, p.out, p.m, p.n,
                       pl.ks, p.o_stride);
  return ss_host::launch_status("w4a16 split-K reduce");
}

template <typename T, int MT, int NS, int ST>
int launch_w4a16_skinny_st(const W4Params& p, const W4Plan& pl, hipStream_t stream) {
  // stages in flight: two, or four for four weight tiles of fewer than eight stages
  // (A B B A at m = 5..16: two against four, 4096 x 4096 5.05 vs 5.50 us at m = 5, 5.25
  // vs 5.61 at m = 8, 4096 x 6144 7.24 vs 7.38 at m = 8; four tiles of 4096 x 14336 12.2
  // vs 11.7 us at m = 5 with two)
  constexpr int P4 = 4 < ST ? 4 : ST;
  constexpr int P2 = 2 < ST ? 2 : ST;
  // 16-wave workgroups get 128 registers a lane; up to 8 waves, 256
  auto launch = [&](auto kern) {
    static bool attr_set = false;  // per instantiation; the attribute is process-wide
    if (!attr_set) {
      if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kSkinnyLdsMax) !=
          hipSuccess) {
        ss_host::set_error("w4a16 gemm: cannot reserve %d bytes of LDS", (int)kSkinnyLdsMax);
        return SS_ERR_UNSUPPORTED;
      }
      attr_set = true;
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)pl.n_tiles, (unsigned)pl.m_blocks), dim3((unsigned)(64 * pl.kw)), pl.lds,
                       stream, p);
    return ss_host::launch_status("w4a16 gemm (skinny)");
  };
  if (pl.kw > 8) {
    if constexpr (NS <= 2) return launch(w4a16_skinny_kernel<T, MT, NS, ST, ST >= 8 ? P2 : P4, 1024>);
    ss_host::set_error("w4a16 gemm: skinny plan with %d waves and %d weight tiles", pl.kw, NS);
    return SS_ERR_UNSUPPORTED;
  }
  return launch(w4a16_skinny_kernel<T, MT, NS, ST, NS >= 4 && ST < 8 ? P4 : P2, 512>);
}

template <typename T, int MT>
int launch_w4a16_skinny_mt(const W4Params& p, const W4Plan& pl, hipStream_t stream) {
  if (pl.ns == 4) {
    if (pl.st == 4) return launch_w4a16_skinny_st<T, MT, 4, 4>(p, pl, stream);
    ss_host::set_error("w4a16 gemm: skinny plan with 4 weight tiles and %d stages", pl.st);
    return SS_ERR_UNSUPPORTED;
  }
  if (pl.ns == 2) {
    switch (pl.st) {
      case 1: return launch_w4a16_skinny_st<T, MT, 2, 1>(p, pl, stream);
      case 2: return launch_w4a16_skinny_st<T, MT, 2, 2>(p, pl, stream);
      case 4: return launch_w4a16_skinny_st<T, MT, 2, 4>(p, pl, stream);
      default: break;
    }
  } else {
    switch (pl.st) {
      case 1: return launch_w4a16_skinny_st<T, MT, 1, 1>(p, pl, stream);
      case 2: return launch_w4a16_skinny_st<T, MT, 1, 2>(p, pl, stream);
      case 4: return launch_w4a16_skinny_st<T, MT, 1, 4>(p, pl, stream);
      case 8: return launch_w4a16_skinny_st<T, MT, 1, 8>(p, pl, stream);
      default: break;
    }
  }
  ss_host::set_error("w4a16 gemm: skinny plan with %d weight tiles and %d stages", pl.ns, pl.st);
  return SS_ERR_UNSUPPORTED;
}

// at most 8 waves of 2048 keys and 4 activation rows
constexpr int kNarrowLdsMax = 160 * 1024;

template <typename T, int MR, int J, int W, int SD>
int launch_w4a16_narrow(const W4Params& p, const W4Plan& pl, hipStream_t stream) {
  static bool attr_set = false;  // per instantiation; the attribute is process-wide
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)w4a16_narrow_kernel<T, MR, J, W, SD>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, kNarrowLdsMax) != hipSuccess) {
      ss_host::set_error("w4a16 gemm: cannot reserve %d bytes of LDS", kNarrowLdsMax);
      return SS_ERR_UNSUPPORTED;
    }
    attr_set = true;
  }
  hipLaunchKernelGGL((w4a16_narrow_kernel<T, MR, J, W, SD>), dim3((unsigned)pl.n_tiles),
                     dim3((unsigned)(64 * (p.k / (512 * W)))), pl.lds, stream, p);
  return ss_host::launch_status("w4a16 gemm (narrow)");
}

template <typename T, int MR, int SD>
int launch_w4a16_narrow_sd(const W4Params& p, const W4Plan& pl, hipStream_t stream) {
  if (p.k <= 8192) return launch_w4a16_narrow<T, MR, 4, 2, SD>(p, pl, stream);
  return launch_w4a16_narrow<T, MR, 4, 4, SD>(p, pl, stream);
}

template <typename T, int MR>
int launch_w4a16_narrow_mr(const W4Params& p, const W4Plan& pl, hipStream_t stream) {
  if (p.sdt == SS_DTYPE_F16) return launch_w4a16_narrow_sd<T, MR, SS_DTYPE_F16>(p, pl, stream);
  if (p.sdt == SS_DTYPE_BF16) return launch_w4a16_narrow_sd<T, MR, SS_DTYPE_BF16>(p, pl, stream);
  return launch_w4a16_narrow_sd<T, MR, SS_DTYPE_F32>(p, pl, stream);
}

template <typename T, int NS, int SD>
int launch_w4a16_wide_sd(const W4Params& p, const W4Plan& pl, float* part, hipStream_t stream) {
  auto kern = w4a16_wide_kernel<T, kWideMT, NS, kWideWV, SD>;
  static bool attr_set = false;  // per instantiation; the attribute is process-wide
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kWideLdsMax) !=
        hipSuccess) {
      ss_host::set_error("w4a16 gemm: cannot reserve %d bytes of LDS", (int)kWideLdsMax);
      return SS_ERR_UNSUPPORTED;
    }
    attr_set = true;
  }
  const int64_t pairs = (int64_t)pl.ks * pl.n_tiles;
  const int64_t grid = (pairs + 7) / 8 * 8 * pl.m_blocks;
  if (grid > 0x7fffffff || pl.ns != NS || pl.lds != wide_lds_bytes(NS, pl.kchunk) || pl.kchunk % kWidePF) {
    ss_host::set_error("w4a16 gemm: wide plan of %lld workgroups, %zu LDS bytes", (long long)grid, pl.lds);
    return SS_ERR_UNSUPPORTED;
  }
  // two ranges (whole 16-byte row chunks, N % 4 == 0): the second range to finish a tile
  // adds the partials itself (C5 gate at m = 256: no reduce launch)
  const bool fused = pl.ks == 2 && p.n % 4 == 0;
  unsigned long long* const arrivals = fused ? (unsigned long long*)((char*)part + tile_part_bytes(pl, p.m, p.n)) : nullptr;
  const unsigned long long tag = fused ? next_arrival_tag() : 0ull;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * kWideWV), pl.lds, stream, p, part, arrivals, tag, pl.kchunk,
                     pl.ks, pl.n_tiles, pl.m_blocks);
  int st = ss_host::launch_status("w4a16 gemm (wide)");
  if (st != SS_OK || pl.ks == 1 || fused) return st;
  const bool vec = p.n % 4 == 0;
  const int64_t threads = (int64_t)p.m * (vec ? p.n / 4 : p.n);
  const unsigned blocks = (unsigned)((threads + 255) / 256);
  if (vec)
    hipLaunchKernelGGL((w4a16_splitk_reduce_kernel<T, 4>), dim3(blocks), dim3(256), 0, stream, part, p.out, p.m, p.n,
                       pl.ks, p.o_stride);
  else
    hipLaunchKernelGGL((w4a16_splitk_reduce_kernel<T, 1>), dim3(blocks), dim3(256), 0, stream, part, p.out, p.m, p.n,
                       pl.ks, p.o_stride);
  return ss_host::launch_status("w4a16 split-K reduce");
}

template <typename T>
int launch_w4a16_typed(const W4Params& p, const W4Plan& pl, float* part, hipStream_t stream) {
  if (pl.widek) {
    if (pl.ns == 1) {
      if (p.sdt == SS_DTYPE_F16) return launch_w4a16_wide_sd<T, 1, SS_DTYPE_F16>(p, pl, part, stream);
      if (p.sdt == SS_DTYPE_BF16) return launch_w4a16_wide_sd<T, 1, SS_DTYPE_BF16>(p, pl, part, stream);
      return launch_w4a16_wide_sd<T, 1, SS_DTYPE_F32>(p, pl, part, stream);
    }
    if (p.sdt == SS_DTYPE_F16) return launch_w4a16_wide_sd<T, kWideNS, SS_DTYPE_F16>(p, pl, part, stream);
    if (p.sdt == SS_DTYPE_BF16) return launch_w4a16_wide_sd<T, kWideNS, SS_DTYPE_BF16>(p, pl, part, stream);
    return launch_w4a16_wide_sd<T, kWideNS, SS_DTYPE_F32>(p, pl, part, stream);
  }
  if (pl.narrow == 1) return launch_w4a16_narrow_mr<T, 1>(p, pl, stream);
  if (pl.narrow == 2) return launch_w4a16_narrow_mr<T, 2>(p, pl, stream);
  if (pl.narrow == 4) return launch_w4a16_narrow_mr<T, 4>(p, pl, stream);
  if (pl.skinny) return launch_w4a16_skinny_mt<T, 1>(p, pl, stream);
  if (pl.tile) {
    // A grid of one workgroup per CU at most (m <= 64 but the widest linears) takes eight
    // waves of half the rows each: two waves per SIMD instead of one, so one wave's MFMAs
    // overlap the other's unpack, fold and staging (C5 at m = 32: 5-6 % faster, m = 64:
    // 1-3 %). Larger grids keep four waves: two of their workgroups share a CU (gate_up at
    // m = 32 and 64 took 11-17 % longer with eight, m = 256 3-10 %).
    const int64_t grid = ((int64_t)pl.ks * pl.n_tiles + 7) / 8 * 8 * pl.m_blocks;
    const bool eight = grid <= ss_host::device_cu_count();
    if (pl.mt == 1) return launch_w4a16_tile<T, 1, 2, 2, 4>(p, pl, part, stream);
    if (pl.mt == 2)
      return eight ? launch_w4a16_tile<T, 2, 1, 2, 8>(p, pl, part, stream)
                   : launch_w4a16_tile<T, 2, 2, 2, 4>(p, pl, part, stream);
    return eight ? launch_w4a16_tile<T, 4, 1, 2, 8>(p, pl, part, stream)
                 : launch_w4a16_tile<T, 4, 2, 2, 4>(p, pl, part, stream);
  }
  if (pl.gemv) {
    if (p.k <= 8192)
      hipLaunchKernelGGL((w4a16_gemv_kernel<T, 1, 8>), dim3((unsigned)pl.n_tiles),
                         dim3((unsigned)(64 * (p.k / 1024))), pl.lds, stream, p);
    else
      hipLaunchKernelGGL((w4a16_gemv_kernel<T, 1, 16>), dim3((unsigned)pl.n_tiles),
                         dim3((unsigned)(64 * (p.k / 2048))), pl.lds, stream, p);
    return ss_host::launch_status("w4a16 gemv");
  }
  if (pl.xlds) return launch_w4a16_x<T, 1, 1, 4, true>(p, pl, stream);
  if (pl.mt == 1 && pl.ns == 4) return launch_w4a16_x<T, 1, 4, 2, false>(p, pl, stream);
  if (pl.mt == 1) return launch_w4a16_x<T, 1, 2, 2, false>(p, pl, stream);
  if (pl.mt == 2) return launch_w4a16_x<T, 2, 2, 2, false>(p, pl, stream);
  return launch_w4a16_x<T, 4, 2, 1, false>(p, pl, stream);
}

}  // namespace
}  // namespace ss

namespace {
bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_w4a16(const char* who, int64_t m, int64_t n, int64_t k, int g, int act_dtype, int scale_dtype) {
  if (m < 0 || n < 0 || k < 0) {
    ss_host::set_error("%s: negative extent (m=%lld n=%lld k=%lld)", who, (long long)m, (long long)n, (long long)k);
    return SS_ERR_INVALID;
  }
  if (g <= 0 || g % 8 != 0) {
    ss_host::set_error("%s: group_size must be a positive multiple of 8, got %d", who, g);
    return SS_ERR_INVALID;
  }
  if (k % g != 0) {
    ss_host::set_error("%s: in_features %lld not divisible by group_size %d", who, (long long)k, g);
    return SS_ERR_INVALID;
  }
  if (m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff || m * n > ((int64_t)1 << 40)) {
    ss_host::set_error("%s: extents too large", who);
    return SS_ERR_UNSUPPORTED;
  }
  if (act_dtype != SS_DTYPE_BF16 && act_dtype != SS_DTYPE_F16 && act_dtype != SS_DTYPE_F32) {
    ss_host::set_error("%s: activation dtype code %d not supported", who, act_dtype);
    return SS_ERR_UNSUPPORTED;
  }
  if (scale_dtype != SS_DTYPE_BF16 && scale_dtype != SS_DTYPE_F16 && scale_dtype != SS_DTYPE_F32) {
    ss_host::set_error("%s: scale dtype code %d not supported", who, scale_dtype);
    return SS_ERR_UNSUPPORTED;
  }
  return SS_OK;
}
}  // namespace

extern "C" int ss_w4a16_workspace_size(int64_t m, int64_t n, int64_t k, int group_size, int act_dtype,
                                       int64_t* bytes) {
  int st = check_w4a16("w4a16 workspace", m, n, k, group_size, act_dtype, SS_DTYPE_F16);
  if (st != SS_OK) return st;
  if (!bytes) {
    ss_host::set_error("w4a16 workspace: null output pointer");
    return SS_ERR_INVALID;
  }
  const ss::W4Plan pl = ss::plan_w4a16(m, n, k, group_size, act_dtype != SS_DTYPE_F32);
  *bytes = pl.fast ? ss::tile_workspace_bytes(pl, m, n) : 0;
  return SS_OK;
}

extern "C" int ss_w4a16_gemm(const void* x, void* out, const int32_t* qweight, const void* scales,
                             const int32_t* qzeros, int64_t m, int64_t n, int64_t k, int group_size,
                             int64_t x_stride, int64_t o_stride, int act_dtype, int scale_dtype,
                             void* workspace, int64_t workspace_bytes, void* stream) {
  const char* who = "w4a16 gemm";
  int st = check_w4a16(who, m, n, k, group_size, act_dtype, scale_dtype);
  if (st != SS_OK) return st;
  if (m == 0 || n == 0) return SS_OK;
  if (!x || !out || !qweight || !scales || !qzeros) {
    ss_host::set_error("%s: null pointer", who);
    return SS_ERR_INVALID;
  }
  if (x_stride < k || o_stride < n) {
    ss_host::set_error("%s: row strides (x %lld, out %lld) shorter than the rows", who, (long long)x_stride,
                       (long long)o_stride);
    return SS_ERR_INVALID;
  }
  ss::W4Params p = {};
  p.x = x;
  p.out = out;
  p.qw = (const uint32_t*)qweight;
  p.sc = scales;
  p.qz = qzeros;
  p.x_stride = x_stride;
  p.o_stride = o_stride;
  p.m = (int)m;
  p.n = (int)n;
  p.k = (int)k;
  p.g = group_size;
  p.groups = (int)(k / group_size);
  p.sdt = scale_dtype;
  const bool act16 = act_dtype != SS_DTYPE_F32;
  ss::W4Plan pl = ss::plan_w4a16(m, n, k, group_size, act16);
  if (pl.fast && (!aligned16(x) || x_stride % 8 != 0 || !aligned16(qweight))) pl.fast = false;
  // activation fragments are addressed by 32-bit byte offsets within a 64-row block
  if (pl.fast && ((int64_t)63 * x_stride + k) * 2 >= ((int64_t)1 << 31)) pl.fast = false;
  // scale and zero-point offsets are 32-bit byte offsets
  if (pl.fast && n * (k / group_size) * 4 >= ((int64_t)1 << 31)) pl.fast = false;
  if (pl.fast && (pl.tile || pl.widek) && pl.ks > 1) {
    // the K split needs the workspace ss_w4a16_workspace_size reports; without it
    // (or unaligned) the untiled MFMA kernel runs, which needs none
    const int64_t need = ss::tile_workspace_bytes(pl, m, n);
    if (!workspace || workspace_bytes < need || !aligned16(workspace)) {
      const bool fast = pl.fast;
      pl = ss::plan_w4a16(m, n, k, group_size, act16, false);
      pl.fast = pl.fast && fast;
    }
  }
  hipStream_t s = (hipStream_t)stream;
  if (!pl.fast) {
    const int64_t total = m * n;
    const int64_t blocks = (total + 255) / 256;
    if (blocks > 0x7fffffff) {
      ss_host::set_error("%s: generic path grid too large", who);
      return SS_ERR_UNSUPPORTED;
    }
    if (act_dtype == SS_DTYPE_BF16)
      hipLaunchKernelGGL((ss::w4a16_generic_kernel<ss::bf16_t>), dim3((unsigned)blocks), dim3(256), 0, s, p);
    else if (act_dtype == SS_DTYPE_F16)
      hipLaunchKernelGGL((ss::w4a16_generic_kernel<ss::f16_t>), dim3((unsigned)blocks), dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL((ss::w4a16_generic_kernel<float>), dim3((unsigned)blocks), dim3(256), 0, s, p);
    return ss_host::launch_status("w4a16 gemm (generic)");
  }
  if (pl.m_blocks > 65535) {
    ss_host::set_error("%s: %lld activation rows exceed the grid", who, (long long)m);
    return SS_ERR_UNSUPPORTED;
  }
  p.kw = pl.kw;
  float* part = (float*)workspace;
  if (act_dtype == SS_DTYPE_BF16) return ss::launch_w4a16_typed<ss::bf16_t>(p, pl, part, s);
  return ss::launch_w4a16_typed<ss::f16_t>(p, pl, part, s);
}
