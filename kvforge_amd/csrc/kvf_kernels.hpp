// kvf_kernels.hpp - split-KV decode attention for gfx950 (MI355X).
//
// One decode step for one layer: a single query vector per head attends to n
// cached tokens, reading every cached byte once. Functionally this is the
// reference's decode_partial / decode_merge (runtime/kvf_kernels.cuh:124-306);
// the mapping onto CDNA4 is this file's own:
//
//   * A 64-lane wavefront consumes 16-token tiles. Lane l sits in lane-row
//     r = l/16 at column c = l%16.
//   * QK^T is an MFMA contraction over the head dimension with the K tile as
//     operand A (token = column c) and the query as operand B (query head =
//     c mod G, every head replicated 16/G times). The 16x16 result leaves in
//     lane l the scores of tokens 4r..4r+3 for query head c mod G.
//   * That is exactly the A-operand layout of the PV MFMA (head = c, tokens
//     4r+j), so softmax weights go from the first MFMA to the second with no
//     cross-lane movement. V is loaded so that lane l holds tokens 4r..4r+3
//     of column block c, which is exactly PV's B operand.
//   * Quantized K feeds the MFMA as exact binary16 codes; each quantization
//     group accumulates separately and its (scale, zero) is applied to the
//     16x16 fp32 result, so scores are fp32-exact up to summation order. The
//     query enters as a binary16 hi/lo pair (two MFMAs), ~22 bits.
//   * V is dequantized to binary16 with one fused multiply-add per element
//     pair (v_pk_fma_f16); softmax weights enter PV as a binary16 hi/lo pair.
//   * Online softmax keeps one running max per head for the whole wave and
//     only rescales when a score exceeds it by more than TAU (log2 units): a
//     wave-uniform, rarely taken branch. The exact max is tracked beside it,
//     so partials report the true max as the reference does.
//   * Loads are issued U tiles ahead (nontemporal, 4-16 B per lane); paged
//     tiles never straddle a page (16 | page size), so the block-table lookup
//     is one scalar load per tile.
//   * Waves of a workgroup combine through LDS; splits combine in
//     decode_merge (log-sum-exp), or the workgroup writes the normalised
//     output directly when splits == 1.
#pragma once

#include "kvf_abi.h"
#include "kvf_registry.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kvf {
namespace gfx950 {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int TILE = 16;       // tokens per wavefront step
constexpr float TAU = 8.0f;    // rescale threshold, log2 units
constexpr uint32_t MAGIC = 0x64646464u; // byte 0x64 -> binary16 1024 + b

template <int FMT> constexpr int bits_of() {
  return FMT == FMT_F16 ? 16 : FMT == FMT_INT8 ? 8 : 4;
}

// Lane geometry of one (format, head dimension, quantization group).
template <int FMT, int D, int GQ> struct Geo {
  static constexpr int BITS = bits_of<FMT>();
  static constexpr int ROW = D * BITS / 8;                 // bytes per cached row
  static constexpr int GRP = FMT == FMT_F16 ? D : GQ;      // elements per scale group
  // QK side: a "piece" is one load per lane; the four lane-rows of a piece
  // cover 4*W consecutive bytes of each of the 16 tokens, inside one group.
  static constexpr int W = FMT == FMT_F16 ? 16 : (GRP * BITS / 32 < 16 ? GRP * BITS / 32 : 16);
  static constexpr int P = ROW / (4 * W);                  // pieces per row
  static constexpr int EP = W * 8 / BITS;                  // elements per lane per piece
  static constexpr int SPP = EP / 8;                       // x32 MFMA steps per piece
  static constexpr int KSTEPS = P * SPP;                   // = D / 32
  static constexpr int NG = D / GRP;                       // scale groups per row
  // PV side: lane holds EV elements (one column block) of 4 tokens.
  static constexpr int EV = D / 16;
  static constexpr int WV = EV * BITS / 8;                 // bytes per token per lane
  static constexpr int WVW = WV >= 4 ? WV / 4 : 1;         // 32-bit words per token
  static constexpr int MW = NG;                            // meta words per row
  static_assert(D == 64 || D == 128, "head dimension");
  static_assert(KSTEPS == D / 32, "piece geometry");
  static_assert(P * 4 * W == ROW, "pieces tile the row");
};

__device__ __forceinline__ uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
  return __builtin_amdgcn_perm(s0, s1, sel);
}

__device__ __forceinline__ half2_t as_h2(uint32_t w) { return __builtin_bit_cast(half2_t, w); }
__device__ __forceinline__ uint32_t as_u(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// Streaming loads of NB bytes (every K/V byte is used once).
template <int NB> struct Raw { uint32_t w[NB >= 4 ? NB / 4 : 1]; };

template <int NB>
__device__ __forceinline__ void load_stream(const unsigned char *p, Raw<NB> &r) {
  if constexpr (NB == 16) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
    r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
  } else if constexpr (NB == 8) {
    const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t *>(p));
    r.w[0] = v.x; r.w[1] = v.y;
  } else if constexpr (NB == 4) {
    r.w[0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p));
  } else {
    static_assert(NB == 2, "load width");
    r.w[0] = __builtin_nontemporal_load(reinterpret_cast<const uint16_t *>(p));
  }
}

// Order in which a lane's converted binary16 values hold its elements, per
// 32-bit word of packed codes. int4 splits even and odd nibbles.
template <int FMT> __device__ __host__ constexpr int slot_elem(int i) {
  if constexpr (FMT == FMT_INT4) {
    constexpr int ord[8] = {0, 2, 4, 6, 1, 3, 5, 7};
    return (i / 8) * 8 + ord[i % 8];
  } else {
    return i;
  }
}

// Raw K words of one piece -> binary16 A-operand values (exact for codes).
template <int FMT, int EP>
__device__ __forceinline__ void k_to_half(const uint32_t *w, uint32_t (&h)[EP / 2]) {
  const half2_t k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
  if constexpr (FMT == FMT_F16) {
#pragma unroll
    for (int i = 0; i < EP / 2; ++i) h[i] = w[i];
  } else if constexpr (FMT == FMT_INT8) {
#pragma unroll
    for (int i = 0; i < EP / 4; ++i) {
      h[2 * i] = as_u(as_h2(perm(MAGIC, w[i], 0x04010400u)) - k1024);
      h[2 * i + 1] = as_u(as_h2(perm(MAGIC, w[i], 0x04030402u)) - k1024);
    }
  } else {
#pragma unroll
    for (int i = 0; i < EP / 8; ++i) {
      const uint32_t lo = w[i] & 0x0F0F0F0Fu;
      const uint32_t hi = (w[i] >> 4) & 0x0F0F0F0Fu;
      h[4 * i + 0] = as_u(as_h2(perm(MAGIC, lo, 0x04010400u)) - k1024);
      h[4 * i + 1] = as_u(as_h2(perm(MAGIC, lo, 0x04030402u)) - k1024);
      h[4 * i + 2] = as_u(as_h2(perm(MAGIC, hi, 0x04010400u)) - k1024);
      h[4 * i + 3] = as_u(as_h2(perm(MAGIC, hi, 0x04030402u)) - k1024);
    }
  }
}

// Element e of tokens A and B of a lane's V column block, as a binary16 pair
// (A low, B high), dequantised with the pair's (scale, zero).
template <int FMT, int EV>
__device__ __forceinline__ uint32_t v_pair(const uint32_t *ta, const uint32_t *tb, int e,
                                           half2_t sc, half2_t z) {
  if constexpr (FMT == FMT_F16) {
    return perm(tb[e / 2], ta[e / 2], (e & 1) ? 0x07060302u : 0x05040100u);
  } else {
    const half2_t k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
    uint32_t x;
    if constexpr (FMT == FMT_INT8) {
      const int k = e & 3;
      x = perm(tb[e / 4], ta[e / 4], (k < 2) ? 0x05010400u : 0x07030602u);
      x = perm(MAGIC, x, (k & 1) ? 0x04030402u : 0x04010400u);
    } else {
      // nibble e: even e are the low nibbles of byte e/2, odd e the high
      const uint32_t a = (e & 1) ? (ta[0] >> 4) & 0x0F0F0F0Fu : ta[0] & 0x0F0F0F0Fu;
      const uint32_t b = (e & 1) ? (tb[0] >> 4) & 0x0F0F0F0Fu : tb[0] & 0x0F0F0F0Fu;
      const int k = (e >> 1) & 3; // byte index
      x = perm(b, a, (k < 2) ? 0x05010400u : 0x07030602u);
      x = perm(MAGIC, x, (k & 1) ? 0x04030402u : 0x04010400u);
    }
    const half2_t c = as_h2(x) - k1024;
    return as_u(__builtin_elementwise_fma(c, sc, z));
  }
}

// Extension fields (variable lengths, binary16 q/out); all null by default.
struct Ext {
  const int *seq_lens = nullptr;
  const _Float16 *q16 = nullptr;
  _Float16 *out16 = nullptr;
};

// Row of (b, h, t) in the cache, as the reference defines it
// (runtime/kvf_kernels.cuh:51-64). For paged layouts `page` is the page that
// holds t (one per 16-token tile).
template <int ORD, bool PAGED>
__device__ __forceinline__ long long tile_row(const Args &a, int b, int h, int t, long long page) {
  if constexpr (!PAGED) {
    return ORD == ORD_HEAD ? ((long long)b * a.Hkv + h) * a.n + t
                           : ((long long)b * a.n + t) * a.Hkv + h;
  } else {
    const int bt = 1 << a.block_shift;
    const long long base = page * a.Hkv * bt;
    return ORD == ORD_HEAD ? base + (long long)h * bt + (t & (bt - 1))
                           : base + (long long)(t & (bt - 1)) * a.Hkv + h;
  }
}

template <int FMT, int D, int GQ, int U, int ORD, bool PAGED>
__global__ void __launch_bounds__(512)
decode_partial(const Args a, const Ext x, const int G, const int final_out) {
  using Gm = Geo<FMT, D, GQ>;
  constexpr int P = Gm::P, EP = Gm::EP, W = Gm::W, SPP = Gm::SPP, KSTEPS = Gm::KSTEPS;
  constexpr int NG = Gm::NG, EV = Gm::EV, WV = Gm::WV, WVW = Gm::WVW;
  constexpr int ROW = Gm::ROW;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = a.warps;
  const int r = lane >> 4;   // lane-row
  const int c = lane & 15;   // column

  const int split = blockIdx.x;
  const int hb = blockIdx.y;
  const int b = blockIdx.z;
  const int gq = a.H / a.Hkv;
  const int hkv = G > 1 ? hb : hb / gq;
  const int my_head = c % G;              // packed head index of this lane
  const int hq_lane = G > 1 ? hkv * G + my_head : hb;

  const int len = x.seq_lens ? x.seq_lens[b] : a.n;
  const int chunk = (len + a.splits - 1) / a.splits;
  const int t0 = split * chunk;
  const int t1 = min(len, t0 + chunk);
  const int tile_first = t0 / TILE;
  const int n_tiles = t1 > t0 ? (t1 - 1) / TILE - tile_first + 1 : 0;

  // ---- query: binary16 hi/lo in the B-operand layout, group sums ----------
  half8_t qhi[KSTEPS], qlo[KSTEPS];
  float qs[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) qs[g] = 0.f;
  {
    const long long qbase = ((long long)b * a.H + hq_lane) * D;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int d0 = p * 4 * EP + r * EP;
      const int grp = (p * 4 * EP) / Gm::GRP;
#pragma unroll
      for (int m = 0; m < SPP; ++m) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int d = d0 + slot_elem<FMT>(8 * m + i);
          float qv = x.q16 ? (float)x.q16[qbase + d] : a.q[qbase + d];
          qv *= a.scale_log2;
          const _Float16 hi = (_Float16)qv;
          const _Float16 lo = (_Float16)(qv - (float)hi);
          qhi[p * SPP + m][i] = hi;
          qlo[p * SPP + m][i] = lo;
          qs[grp] += qv;
        }
      }
    }
  }
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    qs[g] += __shfl_xor(qs[g], 16);
    qs[g] += __shfl_xor(qs[g], 32);
  }

  // ---- per-lane state ------------------------------------------------------
  float4_t acc[EV];
#pragma unroll
  for (int e = 0; e < EV; ++e) acc[e] = (float4_t){0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;  // per head, identical across the lanes of a head
  float m_true = -INFINITY; // exact max of this lane's scores
  float l_sum = 0.f;

  const unsigned char *kbase = a.k;
  const unsigned char *vbase = a.v;
  const uint32_t *kmeta = reinterpret_cast<const uint32_t *>(a.k_meta);
  const uint32_t *vmeta = reinterpret_cast<const uint32_t *>(a.v_meta);
  const int rstride = ORD == ORD_HEAD ? 1 : a.Hkv; // rows between tokens of a tile
  const int vgroup = (c * EV) / Gm::GRP;           // scale group of this lane's V block

  const int n_iter = (n_tiles + nw * U - 1) / (nw * U);
  for (int it = 0; it < n_iter; ++it) {
    Raw<W> kraw[U][P];
    Raw<WV> vraw[U][4];
    uint32_t kmw[U][4][NG];
    uint32_t vmw[U][4];
    int tt[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int ti = wave + nw * (it * U + u);
      tt[u] = ti < n_tiles ? (tile_first + ti) * TILE : -1;
      if (tt[u] >= 0) {
        const int tbase = tt[u];
        long long page = 0;
        if constexpr (PAGED)
          page = a.block_table[(long long)b * a.max_blocks + (tbase >> a.block_shift)];
        const long long row0 = tile_row<ORD, PAGED>(a, b, hkv, tbase, page);
        const int lo_t = max(t0 - tbase, 0);
        const int hi_t = min(t1 - tbase, TILE) - 1;
        // K: token column c
        const int tk = min(max(c, lo_t), hi_t);
        const unsigned char *kp = kbase + (row0 + (long long)tk * rstride) * ROW + r * W;
#pragma unroll
        for (int p = 0; p < P; ++p) load_stream<W>(kp + p * 4 * W, kraw[u][p]);
        // V and meta: tokens 4r+j
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int tv = min(max(4 * r + j, lo_t), hi_t);
          const long long rowv = row0 + (long long)tv * rstride;
          load_stream<WV>(vbase + rowv * ROW + c * WV, vraw[u][j]);
          if constexpr (FMT != FMT_F16) {
#pragma unroll
            for (int g = 0; g < NG; ++g) kmw[u][j][g] = kmeta[rowv * NG + g];
            vmw[u][j] = vmeta[rowv * NG + vgroup];
          }
        }
      }
    }

#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (tt[u] < 0) continue; // wave-uniform
      const int tbase = tt[u];
      // ---- scores --------------------------------------------------------
      float4_t cg[NG];
#pragma unroll
      for (int g = 0; g < NG; ++g) cg[g] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < P; ++p) {
        uint32_t hk[EP / 2];
        k_to_half<FMT, EP>(kraw[u][p].w, hk);
        const int grp = (p * 4 * EP) / Gm::GRP;
#pragma unroll
        for (int m = 0; m < SPP; ++m) {
          half8_t av;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const half2_t h2 = as_h2(hk[4 * m + i]);
            av[2 * i] = h2.x;
            av[2 * i + 1] = h2.y;
          }
          cg[grp] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, qhi[p * SPP + m], cg[grp], 0, 0, 0);
          cg[grp] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, qlo[p * SPP + m], cg[grp], 0, 0, 0);
        }
      }
      float s[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v;
        if constexpr (FMT == FMT_F16) {
          v = cg[0][j];
        } else {
          v = 0.f;
#pragma unroll
          for (int g = 0; g < NG; ++g) {
            const half2_t mz = as_h2(kmw[u][j][g]);
            v = fmaf((float)mz.x, cg[g][j], v);
            v = fmaf((float)mz.y, qs[g], v);
          }
        }
        const int t = tbase + 4 * r + j;
        s[j] = (t >= t0 && t < t1) ? v : -INFINITY;
      }
      // ---- online softmax --------------------------------------------------
      const float tmax = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
      m_true = fmaxf(m_true, tmax);
      if (__any(tmax > m_run + TAU)) { // wave-uniform, rare after the first tile
        float cand = fmaxf(m_run, tmax);
        for (int mask = G; mask < 64; mask <<= 1) cand = fmaxf(cand, __shfl_xor(cand, mask));
        const float alpha = cand == -INFINITY ? 1.f : exp2f(m_run - cand);
        l_sum *= alpha;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float aj = __shfl(alpha, 16 * r + ((4 * r + j) % 16));
#pragma unroll
          for (int e = 0; e < EV; ++e) acc[e][j] *= aj;
        }
        m_run = cand;
      }
      float pj[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) pj[j] = exp2f(s[j] - m_run);
      l_sum += (pj[0] + pj[1]) + (pj[2] + pj[3]);
      // weights as a binary16 hi/lo pair: PV then sees ~22-bit weights
      half4_t pa, pb;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pa[j] = (_Float16)pj[j];
        pb[j] = (_Float16)(pj[j] - (float)pa[j]);
      }
      // ---- values ------------------------------------------------------------
      half2_t sc01 = {(_Float16)1.f, (_Float16)1.f}, z01 = {(_Float16)0.f, (_Float16)0.f};
      half2_t sc23 = sc01, z23 = z01;
      if constexpr (FMT != FMT_F16) {
        sc01 = as_h2(perm(vmw[u][1], vmw[u][0], 0x05040100u));
        z01 = as_h2(perm(vmw[u][1], vmw[u][0], 0x07060302u));
        sc23 = as_h2(perm(vmw[u][3], vmw[u][2], 0x05040100u));
        z23 = as_h2(perm(vmw[u][3], vmw[u][2], 0x07060302u));
      }
      // tokens outside [t0, t1) carry weight 0; zero their values too so a
      // non-finite cache entry cannot turn 0 * inf into NaN
      uint32_t vw[4][WVW];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool ok = s[j] != -INFINITY;
#pragma unroll
        for (int w = 0; w < WVW; ++w) vw[j][w] = ok ? vraw[u][j].w[w] : 0u;
      }
#pragma unroll
      for (int e = 0; e < EV; ++e) {
        const uint32_t b01 = v_pair<FMT, EV>(vw[0], vw[1], e, sc01, z01);
        const uint32_t b23 = v_pair<FMT, EV>(vw[2], vw[3], e, sc23, z23);
        half4_t bv;
        bv[0] = as_h2(b01).x;
        bv[1] = as_h2(b01).y;
        bv[2] = as_h2(b23).x;
        bv[3] = as_h2(b23).y;
        acc[e] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, bv, acc[e], 0, 0, 0);
        acc[e] = __builtin_amdgcn_mfma_f32_16x16x16f16(pb, bv, acc[e], 0, 0, 0);
      }
    }
  }

  // ---- wave result: per head (m_run, l, m_true) and O[head][D] ---------------
  l_sum += __shfl_xor(l_sum, 16);
  l_sum += __shfl_xor(l_sum, 32);
  m_true = fmaxf(m_true, __shfl_xor(m_true, 16));
  m_true = fmaxf(m_true, __shfl_xor(m_true, 32));

  extern __shared__ float smem[];
  // layout: sO[nw][G][D], then sM[nw][G][3]
  float *sO = smem;
  float *sM = smem + nw * G * D;
  if (r == 0 && c < G) {
    sM[(wave * G + c) * 3 + 0] = m_run;
    sM[(wave * G + c) * 3 + 1] = l_sum;
    sM[(wave * G + c) * 3 + 2] = m_true;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int hrow = 4 * r + j;
    if (hrow < G) {
#pragma unroll
      for (int e = 0; e < EV; ++e) sO[(wave * G + hrow) * D + c * EV + e] = acc[e][j];
    }
  }
  __syncthreads();

  const int nthreads = nw * 64;
  for (int idx = threadIdx.x; idx < G * D; idx += nthreads) {
    const int hh = idx / D, col = idx % D;
    float M = -INFINITY;
    for (int w2 = 0; w2 < nw; ++w2) M = fmaxf(M, sM[(w2 * G + hh) * 3 + 2]);
    float L = 0.f, O = 0.f;
    if (M != -INFINITY) {
      for (int w2 = 0; w2 < nw; ++w2) {
        const float mr = sM[(w2 * G + hh) * 3 + 0];
        if (mr == -INFINITY) continue;
        const float wgt = exp2f(mr - M);
        L = fmaf(sM[(w2 * G + hh) * 3 + 1], wgt, L);
        O = fmaf(sO[(w2 * G + hh) * D + col], wgt, O);
      }
    }
    const int hq = G > 1 ? hkv * G + hh : hb;
    const long long head = (long long)b * a.H + hq;
    if (final_out) {
      const float res = L > 0.f ? O / L : 0.f;
      if (x.out16) x.out16[head * D + col] = (_Float16)res;
      else a.out[head * D + col] = res;
    } else {
      a.part_o[(head * a.splits + split) * D + col] = O;
      if (col == 0) {
        a.part_ml[(head * a.splits + split) * 2] = M;
        a.part_ml[(head * a.splits + split) * 2 + 1] = L;
      }
    }
  }
}

// Log-sum-exp recombination of the split partials, one wavefront per head
// (runtime/kvf_kernels.cuh:288-306 computes the same with D threads).
template <int D>
__global__ void __launch_bounds__(64) decode_merge(const Args a, const Ext x) {
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int lane = threadIdx.x;
  const long long head = (long long)b * a.H + hq;
  const int S = a.splits;
  const float *ml = a.part_ml + head * S * 2;
  float M = -INFINITY;
  for (int s = lane; s < S; s += 64) M = fmaxf(M, ml[2 * s]);
#pragma unroll
  for (int mask = 1; mask < 64; mask <<= 1) M = fmaxf(M, __shfl_xor(M, mask));
  constexpr int PER = D / 64;
  float O[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) O[i] = 0.f;
  float L = 0.f;
  if (M != -INFINITY) {
    for (int s = 0; s < S; ++s) {
      const float ms = ml[2 * s];
      if (ms == -INFINITY) continue;
      const float w = exp2f(ms - M);
      L = fmaf(ml[2 * s + 1], w, L);
      const float *po = a.part_o + (head * S + s) * D;
#pragma unroll
      for (int i = 0; i < PER; ++i) O[i] = fmaf(po[lane + 64 * i], w, O[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const float res = L > 0.f ? O[i] / L : 0.f;
    if (x.out16) x.out16[head * D + lane + 64 * i] = (_Float16)res;
    else a.out[head * D + lane + 64 * i] = res;
  }
}

template <int FMT, int D, int GQ, int U, int ORD, bool PAGED>
hipError_t launch_group(const Args &a, const Ext &x, int G, bool partial_only,
                        hipStream_t st) {
  const dim3 grid(a.splits, G > 1 ? a.Hkv : a.H, a.B);
  const dim3 block(a.warps * 64);
  const int final_out = (a.splits == 1 && !partial_only) ? 1 : 0;
  const size_t lds = (size_t)a.warps * G * (D + 3) * sizeof(float);
  hipLaunchKernelGGL((decode_partial<FMT, D, GQ, U, ORD, PAGED>), grid, block, lds, st,
                     a, x, G, final_out);
  if (!final_out && !partial_only)
    hipLaunchKernelGGL((decode_merge<D>), dim3(a.H, a.B), dim3(64), 0, st, a, x);
  return hipGetLastError();
}

// Checks what the kernels assume about Args before anything is launched.
inline bool args_ok(const Args &a, int fmt, int D, int G, bool paged) {
  if (a.warps != 4 && a.warps != 8) return false;
  if (a.B < 1 || a.H < 1 || a.Hkv < 1 || a.n < 0 || a.splits < 1) return false;
  if (a.H % a.Hkv != 0) return false;
  if (G > 1 && a.H / a.Hkv != G) return false;
  if (!a.q || !a.k || !a.v || !a.out) return false;
  if (a.splits > 1 && (!a.part_o || !a.part_ml)) return false;
  if (fmt != FMT_F16 && (!a.k_meta || !a.v_meta)) return false;
  if (fmt != FMT_F16) {
    const int gq = 1 << a.group_shift;
    if (a.group_shift < 5 || a.group_shift > 7 || gq > D) return false;
  }
  if (paged && (a.block_shift < 4 || a.block_shift > 12 || !a.block_table || a.max_blocks < 1))
    return false;
  return true;
}

template <int FMT, int D, int G, int U, int ORD, bool PAGED>
hipError_t launch_ext(const Args &a, const Ext &x, bool partial_only, hipStream_t st) {
  if (!args_ok(a, FMT, D, G, PAGED)) return hipErrorInvalidValue;
  if (a.n == 0) return hipErrorInvalidValue;
  if constexpr (FMT == FMT_F16) {
    return launch_group<FMT, D, 0, U, ORD, PAGED>(a, x, G, partial_only, st);
  } else {
    switch (a.group_shift) {
    case 5: return launch_group<FMT, D, 32, U, ORD, PAGED>(a, x, G, partial_only, st);
    case 6: return launch_group<FMT, D, 64, U, ORD, PAGED>(a, x, G, partial_only, st);
    default:
      if constexpr (D >= 128) return launch_group<FMT, D, 128, U, ORD, PAGED>(a, x, G, partial_only, st);
      return hipErrorInvalidValue;
    }
  }
}

} // namespace gfx950

// The registry-facing template (runtime/kvf_kernels.cuh:309-320 signature).
template <int FMT, int D, int G, int U, int ORD, bool PAGED>
hipError_t launch(const Args &a, hipStream_t st) {
  return gfx950::launch_ext<FMT, D, G, U, ORD, PAGED>(a, gfx950::Ext{}, false, st);
}

} // namespace kvf
