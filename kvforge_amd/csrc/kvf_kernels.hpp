// kvf_kernels.hpp - split-KV decode attention for gfx950 (MI355X).
//
// One decode step for one layer: a single query vector per head attends to n
// cached tokens, reading every cached byte once. Functionally this is the
// reference's decode_partial / decode_merge (runtime/kvf_kernels.cuh:124-306);
// the mapping onto CDNA4 is this file's own.
//
// Work unit: a 64-lane wavefront consumes 32-token tiles made of two 16-token
// sub-tiles (tiles are aligned to absolute token positions, so a sub-tile
// never straddles a page of >= 16 tokens). Lane l sits in lane-row r = l/16
// at column c = l%16.
//
// QK^T: per sub-tile, a 16x16x32 binary16 MFMA chain with the K sub-tile as
// operand A (token = MFMA row: lane (r,c) loads token c) and the query as
// operand B. MFMA columns are (quantisation group, query head) pairs: a
// column carries its head's query restricted to the dims of its group, so
// one accumulator yields per-group partial dots; each lane applies its own
// group's (scale, zero) and a DPP row rotation sums the columns of a head.
// The query enters as a binary16 hi/lo pair (~22 bits). When the pairs fill
// at most 8 columns the hi half sits in columns 0-7 and the lo half in 8-15,
// so one MFMA yields both; otherwise hi and lo are two MFMAs.
//
// Quantized codes enter the MFMAs as exact binary16 values: one v_perm
// (int8) or mask (int4) places two codes as subnormals code * 2^-24. K codes
// stay in that form; V codes go on, through one packed binary16 fma, to
// (code - mid) * 2^-10, centred on the format's mid-range and in the normal
// range (PV products of subnormal codes measured less precise, and the
// centring keeps sum p*code*scale and sum p*zero from cancelling; the zero
// points absorb mid * scale). int4 high nibbles are masked in place (code *
// 16): the query slots they meet carry 1/16 and the V dims they fill are
// scaled back with the code scale. Scores of quantized formats are kept in
// units of 2^-24 and the factor is folded into the exp2 argument.
//
// PV: one 16x16x32 MFMA per 16 output dims and tile, the softmax weights as
// operand A (rows = the same (group, head) pairs, hi/lo split like the
// query), V codes as operand B (MFMA k = the 32 tokens of the tile). The V
// scale of a token and group is folded into that row's weight and the zero
// point into a per-row running sum, so V is never dequantised element by
// element; each lane keeps the rows whose group matches its V dims. Where hi
// and lo halves share the MFMA (separate accumulator rows), the lo half
// enters scaled by 2^11: a weight folded with a small V scale would otherwise
// leave its lo half in the binary16 subnormal range and keep ~12 bits.
//
// Streaming: every wave keeps a ring of DEPTH tiles; tile k+DEPTH-1 is
// issued before tile k is consumed. Loads are raw buffer loads through
// per-sub-tile descriptors built in scalar registers: the record count
// stops the loads at the sequence end, and a tile outside the wave's range
// gets zero-length descriptors whose loads return zeros without touching
// memory, so the load stream is unconditional and the compiler's wait counts
// are static. Within a tile both sub-tiles' K go first, then the (scale,
// zero) words, then V, so scores and softmax start before V has arrived.
// The first DEPTH-1 tiles are issued before the query is converted, so the
// two latencies overlap. Head-major rows load as nontemporal; token-major
// rows and their (scale, zero) words use the default cache policy (see
// cpol_kv): a token's words of all KV heads share one line, which the other
// heads' workgroups then find in L2.
//
// Online softmax keeps one running max per head for the whole wave and only
// rescales when a score exceeds it by more than TAU (log2 units): a
// wave-uniform, rarely taken branch. The exact max is tracked beside it, so
// partials report the true max as the reference does. Waves of a workgroup
// combine through LDS; splits combine in decode_merge (log-sum-exp), in the
// last workgroup of a head group when the caller supplies merge counters, or
// the workgroup writes the normalised output directly when splits == 1.
#pragma once

#include "kvf_abi.h"
#include "kvf_ext.hpp"
#include "kvf_registry.h"

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <type_traits>

namespace kvf {
namespace gfx950 {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef int32_t i32x2_t __attribute__((ext_vector_type(2)));
typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int SUB = 16;                  // tokens per sub-tile (MFMA rows)
constexpr int TT = 32;                   // tokens per tile (PV MFMA k)
constexpr float TAU = 8.0f;              // rescale threshold, log2 units
constexpr float CODE_SHIFT = 16384.f;    // 2^14: code * 2^-24 (subnormal) -> code * 2^-10
constexpr float CODE_UNIT = 1024.f;      // 2^10: undoes the codes' scale in the MFMAs
constexpr float SUB_UNIT = 16777216.f;   // 2^24: undoes the subnormal encoding of K codes
constexpr float LO_SCALE = 2048.f;       // 2^11: lo half of a packed softmax weight
constexpr float LO_INV = 1.f / 2048.f;
constexpr float INT4_HI = 16.f;          // high nibbles enter the MFMAs as code * 16
// A quantized kernel's query enters its binary16 hi/lo split multiplied by
// 2^6: the lo half of an element below 4 (in log2 units per score) would be
// a binary16 subnormal, which keeps fewer bits (int4 high-nibble slots, held
// at 1/16, most of all). Scores come out 2^6 larger, which the score unit
// takes back. The query must then stay below 1023 in magnitude after the
// softmax scale (|q| < 8000 at d = 128 with scale 1/sqrt(d)).
constexpr float Q_PRESCALE = 64.f;
// int8 kernels whose weights share one accumulator for hi and lo (more than
// 8 columns) take softmax weights 2^4 larger: p * scale_v is far below 1 and
// its lo half would otherwise be subnormal. The factor is undone in the
// wave's running max (m - 4 for l and O that are 16 times larger), so it
// costs nothing per tile. It bounds an int8 V group's scale at 16 (a range
// of 4080 per group) instead of 256: a weight never exceeds 2^(8+4) * scale.
constexpr float W_LOG2 = 4.f;
// V codes enter the PV MFMA centred on their mid-range, code - mid, and a
// token's zero point becomes zero + mid * scale: the products and the zero
// sum then stay near the output's own magnitude instead of cancelling (int8
// codes 0..255 times scale reach |zero|, and sum p*code*scale and sum
// p*zero nearly cancel in the mean of zero-mean data).
template <int FMT> constexpr float vmid() { return FMT == FMT_INT8 ? 128.f : 8.f; }
constexpr int RSRC_WORD3 = 0x00020000;   // gfx9 raw buffer: 32-bit data format
constexpr int CPOL_NT = 2;               // nontemporal: every byte is used once
// Cache policy of the K/V payload loads. Head-major rows stream as
// nontemporal. Token-major rows (a token's rows of all KV heads side by side,
// each head group reading one row in Hkv) load with the default policy:
// measured on GQA 32/8, d128, 32k tokens, int8:64 stored token-major,
// nontemporal loads took 18.9 us against 16.4 us, and the KV head whose rows
// sit at byte 384 of every 1 KiB token block lagged the others by ~4.5 us.
// The (scale, zero) words follow the same policy: a token's words of all KV
// heads share one line, which the other heads' workgroups then find in L2.
template <int ORD> constexpr int cpol_kv() { return ORD == ORD_TOKEN ? 0 : CPOL_NT; }

// Factor that undoes the code * 16 of int4 high nibbles (odd dims of a
// lane's V block) in the PV accumulators.
template <int FMT> __device__ constexpr float vdim_scale(int e) {
  return FMT == FMT_INT4 && (e & 1) ? 1.f / INT4_HI : 1.f;
}

template <int FMT> constexpr int bits_of() {
  return FMT == FMT_F16 ? 16 : FMT == FMT_INT8 ? 8 : 4;
}

// Bytes of LDS the split kernel's wave combine takes: sO and sM, plus sL for
// the lo halves of packed hi/lo rows when all three fit in 64 KiB.
constexpr int LDS_LIMIT = 65536;
template <int D, int G> constexpr bool hl_lds_fits(int nw) {
  return (2 * nw * G * D + nw * G * 3) * 4 <= LDS_LIMIT;
}
template <int FMT, int D, int GQ, int G> constexpr size_t combine_lds(int nw);

// Tiles kept in flight per wave for the reference's unroll knob U.
template <int U> constexpr int depth_of() { return U == 2 ? 2 : 3; }

// Lane geometry of one (format, head dim, quantisation group, pack size).
template <int FMT, int D, int GQ, int G> struct Geo {
  static constexpr int BITS = bits_of<FMT>();
  static constexpr bool QUANT = FMT != FMT_F16;
  static constexpr int ROW = D * BITS / 8;            // bytes per cached row
  static constexpr int GRP = QUANT ? GQ : D;          // elements per scale group
  static constexpr int NG = D / GRP;                  // scale groups per row
  static constexpr int COLS = G * NG;                 // (group, head) pairs
  static constexpr bool HL = COLS <= 8;               // hi/lo share one MFMA
  static constexpr int PASSES = COLS > 16 ? 2 : 1;
  // K: lane-row r loads CH bytes at r*CH + j*4*CH of its token's row.
  static constexpr int CH = ROW / 4 < 16 ? ROW / 4 : 16;
  static constexpr int NCH = ROW / (4 * CH);
  static constexpr int SPC = CH * 8 / BITS / 8;       // MFMA k-steps per chunk
  static constexpr int KSTEPS = NCH * SPC;            // = D / 32
  // V: lane column c owns dims [c*EV, c*EV+EV) of 8 tokens.
  static constexpr int EV = D / 16;
  static constexpr int VB = EV * BITS / 8;            // bytes per token per lane
  static constexpr int VW = VB >= 4 ? VB / 4 : 1;     // 32-bit words per token
  // G >= 4: the 4 columns of a quad share a group, so lane (r, c) loads the
  // whole meta row of token 4r + c%4 and a quad broadcast hands it around
  static constexpr bool QMETA = QUANT && G >= 4;
  static_assert(D == 64 || D == 128, "head dimension");
  static_assert(G == 1 || G == 2 || G == 4 || G == 8, "pack size");
  static_assert(KSTEPS * 32 == D, "chunk geometry");
  static_assert(NCH * 4 * CH == ROW, "chunks tile the row");
  static_assert(!QUANT || (GQ >= 32 && GQ <= D), "group");
  static_assert(COLS <= 32, "at most two column passes");
};

template <int FMT, int D, int GQ, int G> constexpr size_t combine_lds(int nw) {
  const bool sl = Geo<FMT, D, GQ, G>::HL && hl_lds_fits<D, G>(nw);
  return (size_t)(nw * G * (sl ? 2 * D + 3 : D + 3)) * sizeof(float);
}

__device__ __forceinline__ uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
  return __builtin_amdgcn_perm(s0, s1, sel);
}
__device__ __forceinline__ half2_t as_h2(uint32_t w) { return __builtin_bit_cast(half2_t, w); }
__device__ __forceinline__ float lo_f(uint32_t w) { return (float)as_h2(w).x; }
__device__ __forceinline__ float hi_f(uint32_t w) { return (float)as_h2(w).y; }

// byte k of s1 and byte k of s0, each zero-extended to 16 bits:
// two codes as binary16 subnormals (code * 2^-24)
__device__ __host__ constexpr uint32_t sel_pair(int k) {
  return 0x0c000c00u | ((uint32_t)(4 + k) << 16) | (uint32_t)k;
}

// Rotation by N lanes inside each row of 16 (DPP row_ror).
template <int N> __device__ __forceinline__ float ror16(float x) {
  static_assert(N >= 1 && N <= 15, "rotation");
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x120 + N, 0xF, 0xF, false));
}

// Value of lane l ^ 16 and l ^ 32 through gfx950's permlane swaps (VALU, no
// LDS round trip). permlane16_swap exchanges the odd rows of its first
// operand with the even rows of its second, permlane32_swap the upper half of
// the first with the lower half of the second; with x in both, the partner's
// value sits in the second result for lanes of an even row (resp. the lower
// half) and in the first result otherwise.
__device__ __forceinline__ float xor16(float x) {
  const auto s = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x),
                                                  __builtin_bit_cast(uint32_t, x), false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 16) ? s[0] : s[1]);
}
__device__ __forceinline__ float xor32(float x) {
  const auto s = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x),
                                                  __builtin_bit_cast(uint32_t, x), false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 32) ? s[0] : s[1]);
}

// Sum of x over the columns c' == c (mod G) of the lane's row of 16.
template <int G> __device__ __forceinline__ float sum_head_cols(float x) {
  if constexpr (G <= 1) x += ror16<1>(x);
  if constexpr (G <= 2) x += ror16<2>(x);
  if constexpr (G <= 4) x += ror16<4>(x);
  if constexpr (G <= 8) x += ror16<8>(x);
  return x;
}

// Raw buffer loads of NB bytes at voffset through descriptor `rs`.
template <int NB> struct Raw { uint32_t w[NB >= 4 ? NB / 4 : 1]; };

template <int NB, int CPOL = CPOL_NT>
__device__ __forceinline__ void bload(__amdgpu_buffer_rsrc_t rs, int voff, Raw<NB> &r) {
  if constexpr (NB == 16) {
    const i32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, 0, CPOL);
    r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
  } else if constexpr (NB == 8) {
    const i32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(rs, voff, 0, CPOL);
    r.w[0] = v.x; r.w[1] = v.y;
  } else if constexpr (NB == 4) {
    r.w[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, voff, 0, CPOL);
  } else {
    static_assert(NB == 2, "load width");
    r.w[0] = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rs, voff, 0, CPOL);
  }
}

// Buffer descriptor over [base + off, base + off + bytes). Every field is
// wave-uniform by construction; readfirstlane makes that explicit so the
// descriptor lives in scalar registers (a descriptor the compiler believes
// divergent would wrap every load in a waterfall loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base, long long off,
                                                       uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base) + (uint64_t)off;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
  const uint32_t n = __builtin_amdgcn_readfirstlane(bytes);
  void *ptr = reinterpret_cast<void *>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(ptr, 0, (int)n, RSRC_WORD3);
}

// Order in which a lane's binary16 values hold the 8 elements of one k-step.
// int4: low nibbles of bytes 0, 2, 1, 3, then their high nibbles.
template <int FMT> __device__ __host__ constexpr int slot_elem(int i) {
  if constexpr (FMT == FMT_INT4) return (i & 1) * 4 + ((i >> 1) & 1) * 2 + (i >> 2); // 0 4 2 6 1 5 3 7
  else return i;
}

// Loads of one tile in flight.
template <int FMT, int D, int GQ, int G> struct TileBuf {
  using Gm = Geo<FMT, D, GQ, G>;
  Raw<Gm::CH> k[2][Gm::NCH];                      // sub-tile s, token c
  Raw<Gm::VB> v[8];                               // token tau(r, i)
  // (scale, zero) of K and V for tau(r, i), per pass; with QMETA the word of
  // the lane's group (per pass) of token 4r + c%4 of each sub-tile,
  // broadcast across the quad in compute()
  uint32_t km[Gm::QUANT && !Gm::QMETA ? Gm::PASSES : 1][8];
  uint32_t vm[Gm::QUANT && !Gm::QMETA ? Gm::PASSES : 1][8];
  Raw<Gm::QMETA ? 4 * Gm::PASSES : 4> kmr[2], vmr[2];
};

// Two V codes as byte- or nibble-built binary16 subnormals (code * 2^-24) to
// (code - mid) * 2^-10: one packed binary16 fma, exact (the results are
// integers below 2^8 in magnitude times 2^-10, so normal or zero). Measured
// on gfx950 against the double-precision reference: centred subnormal codes
// left int4:32 at 64k tokens at rel_l2 1.0e-4 and int8:64 with outlier
// channels at 32k at 9e-6; normal-range codes 3.1e-6 and 1.2e-6.
__device__ __forceinline__ uint32_t centre_codes(uint32_t w, float mid) {
  const _Float16 m = (_Float16)(mid * (1.f / CODE_UNIT));
  const half2_t h = as_h2(w) * (half2_t){(_Float16)CODE_SHIFT, (_Float16)CODE_SHIFT} - (half2_t){m, m};
  return __builtin_bit_cast(uint32_t, h);
}

// Broadcast of quad lane I's value to the whole quad (DPP quad_perm).
template <int I> __device__ __forceinline__ uint32_t quad_bcast(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, I * 0x55, 0xF, 0xF, false);
}

// Calls f(std::integral_constant<int, i>) for i = 0 .. N-1.
template <int N, int I = 0, class F> __device__ __forceinline__ void static_for(F &&f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<N, I + 1>(f);
  }
}

// Token of the tile held in slot i of lane-row r for the score and PV
// layouts: sub-tile i/4, row 4r + i%4.
__device__ __forceinline__ int tau(int r, int i) { return (i >> 2) * SUB + 4 * r + (i & 3); }

constexpr int CPOL_SC1 = 16; // buffer-load cache policy: device-coherent (sc1)
constexpr int CPOL_SC0 = 1;  // buffer-load cache policy: skip the CU's L1, served by L2
template <int D, int G, int NW>
__device__ __forceinline__ void merge_heads(const Args &a, const Ext &x, long long head0, bool dry);

// Longest first (Ext::longest_first): workgroup slot k serves the sequence of
// rank k in decreasing length (ties: lower index first), so the longest
// sequences' workgroups are dispatched first and the short ones fill the
// tail. B <= 64: lane i holds sequence i's length; every lane returns the
// same sequence index, and its length in len_k.
__device__ __forceinline__ int longest_first(const int *lens, int B, int k, int &len_k) {
  const int lane = threadIdx.x & 63;
  const int li = lane < B ? lens[lane] : -1;
  int rank = 0;
  for (int j = 0; j < B; ++j) {
    const int lj = __builtin_amdgcn_readlane(li, j);
    rank += (lj > li) || (lj == li && j < lane);
  }
  // the ranks of lanes < B are a permutation of 0..B-1: exactly one matches
  const unsigned long long hit = __ballot(lane < B && rank == k);
  const int idx = (int)__builtin_ctzll(hit);
  len_k = __builtin_amdgcn_readlane(li, idx);
  return idx;
}

// One work item of the split kernel: split `split` of head group `hb` of
// sequence slot `b` (a sequence index, or its rank by length with
// Ext::longest_first). With Ext::queue (decode_persistent), thread 0 claims
// the workgroup's next item while the item's last tiles are in flight and
// leaves the claim in *s_next before the workgroup's combine barrier.
template <int FMT, int D, int GQ, int G, int U, int ORD, bool PAGED, int WPB, bool QUEUE>
__device__ __forceinline__ void decode_item(const Args &a, const Ext &x, const int final_out, const int split,
                                            const int hb, int b, unsigned *s_next) {
  using Gm = Geo<FMT, D, GQ, G>;
  constexpr bool QUANT = Gm::QUANT, HL = Gm::HL, QMETA = Gm::QMETA;
  constexpr int ROW = Gm::ROW, NG = Gm::NG, COLS = Gm::COLS, PASSES = Gm::PASSES;
  constexpr int CH = Gm::CH, NCH = Gm::NCH, SPC = Gm::SPC, KSTEPS = Gm::KSTEPS;
  constexpr int EV = Gm::EV, VB = Gm::VB, VW = Gm::VW, GRP = Gm::GRP;
  constexpr int DEPTH = depth_of<U>();
  constexpr bool HL_LDS = HL && hl_lds_fits<D, G>(WPB);
  constexpr int NQ = HL ? 1 : 2;                   // query operands per k-step
  constexpr float UNIT = QUANT ? SUB_UNIT / Q_PRESCALE : 1.f; // log2 units per score unit
  constexpr float QPS = QUANT ? Q_PRESCALE : 1.f;
  constexpr float WOFF = FMT == FMT_INT8 && !HL ? W_LOG2 : 0.f; // log2 of the weights' extra factor
  constexpr float TAU_S = TAU / UNIT;
  using Buf = TileBuf<FMT, D, GQ, G>;

  // In the persistent loop the thread id passes through an empty asm: the
  // compiler then cannot hoist the lane-derived offsets out of the item loop,
  // where they would stay live across it (256 VGPRs and occupancy 1 instead
  // of the one-item kernel's 205-243 and 2)
  unsigned tid = threadIdx.x;
  if constexpr (QUEUE) asm volatile("" : "+v"(tid));
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr int nw = WPB; // equals a.warps, checked at launch
  const int r = lane >> 4;
  const int c = lane & 15;

  const int gy = G > 1 ? a.Hkv : a.H; // head groups per sequence
  const int gq = a.H / a.Hkv;
  const int hkv = G > 1 ? hb : hb / gq;

  // The split's tiles: with uniform lengths a contiguous chunk, tokens
  // [t0, t1) (runtime/kvf_kernels.cuh:147-150). With per-sequence lengths:
  // - paged: every S-th tile, tiles split, split + S, ... below the
  //   sequence's length, so the tiles and their page ids are known before the
  //   length arrives;
  // - contiguous: a chunk of ceil(len / S) tokens rounded up to whole tiles
  //   (the splits past the sequence's end are empty). The S-th-tile order
  //   put a sequence's S splits on neighbouring tiles, one window of rows
  //   that all of them streamed through together: int8 at 16 splits on a
  //   log-uniform batch of 16 sequences took 127 us against 108 us in chunks.
  // Tile j of the split (j = wave + nw * k for a wave's k-th) starts at token
  // (tile0 + tstep * j) * TT.
  const bool varlen = x.seq_lens != nullptr;
  const bool strided = varlen && PAGED;
  const bool lpt = varlen && x.longest_first && a.B > 1 && a.B <= 64;
  int len = a.n;
  int t0 = 0, t1 = 0, n_tiles = 0, nk = 0;
  int tile0 = strided ? split : 0;
  const int tstep = strided ? a.splits : 1;

  // ---- paged: page ids of this wave's sub-tiles, 64 per batch (lane = sub-tile)
  int vpages = 0;
  const int bs = a.block_shift;
  auto load_pages = [&](int kb32) __attribute__((always_inline)) {
    if constexpr (PAGED) {
      const int kk = kb32 + (lane >> 1);
      const int ti = wave + nw * kk;
      const long long t = (long long)(tile0 + (long long)tstep * ti) * TT + (lane & 1) * SUB;
      int pg = 0;
      // strided: every entry inside the sequence's table row is read without
      // waiting for the length (entries past it are never used: their tiles
      // are not live); contiguous chunks: only the split's own entries
      if (strided ? (t >> bs) < a.max_blocks : (kk < nk && ti < n_tiles && t < len))
        pg = a.block_table[(long long)b * a.max_blocks + (t >> bs)];
      vpages = pg;
    }
  };
  // per-sequence lengths in index order: the first page ids go out before the
  // length is loaded, and the empty asm keeps the compiler from issuing the
  // length's scalar load first (a scalar load's wait covers every scalar load
  // in flight, so the page-table pointer's wait would then wait for it too)
  const bool early_pages = PAGED && strided && !lpt;
  if (early_pages) {
    load_pages(0);
    asm volatile("" ::: "memory");
  }
  if (varlen) {
    if (lpt) b = longest_first(x.seq_lens, a.B, b, len);
    else len = x.seq_lens[b];
  }
  if (strided) {
    t1 = len;
    const int tt = (len + TT - 1) / TT;
    n_tiles = tt > split ? (tt - split + a.splits - 1) / a.splits : 0;
  } else {
    const int per = (len + a.splits - 1) / a.splits;
    const int chunk = varlen ? (per + TT - 1) / TT * TT : per;
    t0 = split * chunk;
    t1 = min(len, t0 + chunk);
    tile0 = t0 / TT;
    n_tiles = t1 > t0 ? (t1 - 1) / TT - tile0 + 1 : 0;
  }
  nk = wave < n_tiles ? (n_tiles - wave + nw - 1) / nw : 0; // this wave's tiles
  if (!early_pages) load_pages(0);

  // (group, head) pair of column c in pass p; HL packs the hi half in
  // columns 0-7 and the lo half in 8-15, columns beyond the pairs stay zero
  auto col_id = [&](int p) __attribute__((always_inline)) { return HL ? (c & 7) : ((p * 16 + c) % COLS); };
  const bool col_live = HL ? (c & 7) < COLS : true;
  const bool col_lo = HL && c >= 8;

  // ---- per-lane constant offsets inside a sub-tile -----------------------------
  const int tstride = ORD == ORD_HEAD ? 1 : a.Hkv; // rows between tokens
  const int koff = c * tstride * ROW + r * CH;
  int voff[4], moff[PASSES][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    voff[i] = (4 * r + i) * tstride * ROW + c * VB;
#pragma unroll
    for (int p = 0; p < PASSES; ++p)
      moff[p][i] = ((4 * r + i) * tstride * NG + (col_id(p) % COLS) / G) * 4;
  }
  // QMETA: the word of the lane's group in the meta row of token 4r + c%4
  // (the 4 columns of a quad share a group)
  int mword[PASSES];
#pragma unroll
  for (int p = 0; p < PASSES; ++p)
    mword[p] = ((4 * r + (c & 3)) * tstride * NG + (col_id(p) % COLS) / G) * 4;


  // ---- issue all loads of wave-tile k into buf ---------------------------------
  // Order: both sub-tiles' K, then the (scale, zero) words, then V. Wait counts
  // are in issue order, so a wave can compute a tile's scores and softmax while
  // its V is still arriving.
  auto issue = [&](Buf &buf, int k) __attribute__((always_inline)) {
    const bool live = k >= 0 && k < nk;
    const int tbase = (tile0 + tstep * (wave + nw * k)) * TT;
    __amdgpu_buffer_rsrc_t rk[2], rv[2], rkm[2], rvm[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int ts = tbase + s * SUB;
      long long row0;
      if constexpr (!PAGED) {
        row0 = ORD == ORD_HEAD ? ((long long)b * a.Hkv + hkv) * a.n + ts
                               : ((long long)b * a.n + ts) * a.Hkv + hkv;
      } else {
        if (s == 0 && (k & 31) == 0 && k > 0) load_pages(k);
        const long long page = live ? __builtin_amdgcn_readlane(vpages, 2 * (k & 31) + s) : 0;
        const int bt = 1 << bs;
        const long long base = page * a.Hkv * bt;
        row0 = ORD == ORD_HEAD ? base + (long long)hkv * bt + (ts & (bt - 1))
                               : base + (long long)(ts & (bt - 1)) * a.Hkv + hkv;
      }
      // tokens this sub-tile may read: up to the sequence end
      const int nv = live ? min(SUB, max(0, len - ts)) : 0;
      const uint32_t dbytes = nv > 0 ? (uint32_t)((nv - 1) * tstride * ROW + ROW) : 0u;
      rk[s] = rsrc(a.k, row0 * ROW, dbytes);
      rv[s] = rsrc(a.v, row0 * ROW, dbytes);
      if constexpr (QUANT) {
        const uint32_t mbytes = nv > 0 ? (uint32_t)(((nv - 1) * tstride + 1) * NG * 4) : 0u;
        rkm[s] = rsrc(a.k_meta, row0 * NG * 4, mbytes);
        rvm[s] = rsrc(a.v_meta, row0 * NG * 4, mbytes);
      }
    }
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int j = 0; j < NCH; ++j) bload<CH, cpol_kv<ORD>()>(rk[s], koff + j * 4 * CH, buf.k[s][j]);
    if constexpr (QUANT) {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        if constexpr (QMETA) {
#pragma unroll
          for (int p = 0; p < PASSES; ++p) {
            Raw<4> t;
            bload<4, cpol_kv<ORD>()>(rkm[s], mword[p], t);
            buf.kmr[s].w[p] = t.w[0];
            bload<4, cpol_kv<ORD>()>(rvm[s], mword[p], t);
            buf.vmr[s].w[p] = t.w[0];
          }
        } else
#pragma unroll
        for (int p = 0; p < PASSES; ++p)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            Raw<4> t;
            bload<4, cpol_kv<ORD>()>(rkm[s], moff[p][i], t);
            buf.km[p][4 * s + i] = t.w[0];
            bload<4, cpol_kv<ORD>()>(rvm[s], moff[p][i], t);
            buf.vm[p][4 * s + i] = t.w[0];
          }
      }
    }
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i) bload<VB, cpol_kv<ORD>()>(rv[s], voff[i], buf.v[4 * s + i]);
  };

  // ---- query loads, then the first DEPTH-1 tiles under them ------------------------
  // The ring is three named buffers picked by compile-time index, so every
  // access has a constant address and the buffers stay in registers.
  Buf buf0, buf1, buf2;
  auto ring = [&](auto I) __attribute__((always_inline)) -> Buf & {
    constexpr int i = decltype(I)::value;
    if constexpr (i == 0) return buf0;
    else if constexpr (i == 1) return buf1;
    else return buf2;
  };
  // query loads: both forms through buffer descriptors over the head group's
  // rows (the form not in use has length 0 and reads zeros), so the load
  // stream has no branch; converted to fp32 where the query is first needed
  Raw<16> qf[KSTEPS][2];
  Raw<16> qh[KSTEPS];
  {
    const long long qrow0 = (long long)b * a.H + (G > 1 ? hkv * G : hb); // first head of the group
    const __amdgpu_buffer_rsrc_t rqf = rsrc(a.q, qrow0 * D * 4, x.q16 ? 0u : (uint32_t)(G * D * 4));
    const __amdgpu_buffer_rsrc_t rqh = rsrc(x.q16, qrow0 * D * 2, x.q16 ? (uint32_t)(G * D * 2) : 0u);
    const int qh_lane = G > 1 ? c % G : 0;
#pragma unroll
    for (int j = 0; j < NCH; ++j)
#pragma unroll
      for (int m = 0; m < SPC; ++m) {
        const int d0 = qh_lane * D + (j * 4 * CH + r * CH) * 8 / Gm::BITS + 8 * m;
        bload<16, 0>(rqf, d0 * 4, qf[j * SPC + m][0]);
        bload<16, 0>(rqf, d0 * 4 + 16, qf[j * SPC + m][1]);
        bload<16, 0>(rqh, d0 * 2, qh[j * SPC + m]);
      }
  }
  static_for<DEPTH - 1>([&](auto Ui) __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    issue(ring(Ui), decltype(Ui)::value);
  });
  __builtin_amdgcn_sched_barrier(0);

  float raw[KSTEPS][8];
#pragma unroll
  for (int ks = 0; ks < KSTEPS; ++ks) {
    const half8_t h = __builtin_bit_cast(half8_t, (u32x4_t){qh[ks].w[0], qh[ks].w[1], qh[ks].w[2], qh[ks].w[3]});
#pragma unroll
    for (int i = 0; i < 8; ++i)
      raw[ks][i] = x.q16 ? (float)h[i] : __builtin_bit_cast(float, qf[ks][i / 4].w[i % 4]);
  }

  // ---- query: binary16 hi/lo B operands, zero outside the column's group ----
  half8_t qb[PASSES][NQ][KSTEPS];
  float qs[PASSES]; // sum of q' over the column's (group, head), score units
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int cg = (col_id(p) % COLS) / G;
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; ++j)
#pragma unroll
      for (int m = 0; m < SPC; ++m) {
        const int ks = j * SPC + m;
        const int dgrp = ((j * 4 * CH + r * CH) * 8 / Gm::BITS + 8 * m) / GRP;
        const bool mine = col_live && dgrp == cg;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float v = mine ? raw[ks][slot_elem<FMT>(i)] * a.scale_log2 : 0.f;
          // int4: slots 4-7 meet high nibbles entered as code * 16
          const float vb = FMT == FMT_INT4 && i >= 4 ? v * (QPS / INT4_HI) : v * QPS;
          const _Float16 hi = (_Float16)vb;
          const _Float16 lo = (_Float16)(vb - (float)hi);
          if constexpr (HL) {
            qb[p][0][ks][i] = col_lo ? lo : hi;
          } else {
            qb[p][0][ks][i] = hi;
            qb[p][NQ - 1][ks][i] = lo;
          }
          sum += v;
        }
      }
    sum += xor16(sum);
    sum += xor32(sum);
    qs[p] = col_lo ? 0.f : sum / UNIT;
  }

  // ---- per-lane state ----------------------------------------------------------
  float4_t acc[PASSES][EV];
#pragma unroll
  for (int p = 0; p < PASSES; ++p)
#pragma unroll
    for (int e = 0; e < EV; ++e) acc[p][e] = (float4_t){0.f, 0.f, 0.f, 0.f};
  float zacc[PASSES];
#pragma unroll
  for (int p = 0; p < PASSES; ++p) zacc[p] = 0.f;
  float m_run = -INFINITY;  // running max, score units; equal across a head's lanes
  float m_neg = INFINITY;   // -m_run in log2 units, plus WOFF
  float m_true = -INFINITY; // exact max of this lane's scores, score units
  float l_sum = 0.f;

  // ---- consume one tile --------------------------------------------------------
  auto compute = [&](Buf &buf, int k, auto mask_tag) __attribute__((always_inline)) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int tbase = (tile0 + tstep * (wave + nw * k)) * TT;
    // per-pass (scale, zero) of tokens tau(r, i) for this lane's group
    uint32_t kmeta[QUANT ? PASSES : 1][8], vmeta[QUANT ? PASSES : 1][8];
    if constexpr (QMETA) {
#pragma unroll
      for (int p = 0; p < PASSES; ++p) {
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const uint32_t ks = buf.kmr[st].w[p], vs = buf.vmr[st].w[p];
          kmeta[p][4 * st + 0] = quad_bcast<0>(ks);
          kmeta[p][4 * st + 1] = quad_bcast<1>(ks);
          kmeta[p][4 * st + 2] = quad_bcast<2>(ks);
          kmeta[p][4 * st + 3] = quad_bcast<3>(ks);
          vmeta[p][4 * st + 0] = quad_bcast<0>(vs);
          vmeta[p][4 * st + 1] = quad_bcast<1>(vs);
          vmeta[p][4 * st + 2] = quad_bcast<2>(vs);
          vmeta[p][4 * st + 3] = quad_bcast<3>(vs);
        }
      }
    } else if constexpr (QUANT) {
#pragma unroll
      for (int p = 0; p < PASSES; ++p)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          kmeta[p][i] = buf.km[p][i];
          vmeta[p][i] = buf.vm[p][i];
        }
    }
    // masked tokens (outside [t0, t1)) carry weight 0; their values are
    // zeroed too, so a non-finite entry outside the chunk cannot leak in
    bool ok[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      ok[i] = true;
      if constexpr (MASK) {
        const int t = tbase + tau(r, i);
        ok[i] = t >= t0 && t < t1;
#pragma unroll
        for (int w = 0; w < VW; ++w) buf.v[i].w[w] = ok[i] ? buf.v[i].w[w] : 0u;
        if constexpr (QUANT) {
#pragma unroll
          for (int p = 0; p < PASSES; ++p) vmeta[p][i] = ok[i] ? vmeta[p][i] : 0u;
        }
      }
    }

    // ---- scores: QK^T over (group, head) columns, per sub-tile ----------------
    float s[8];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      float4_t cq[PASSES];
#pragma unroll
      for (int p = 0; p < PASSES; ++p) cq[p] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
#pragma unroll
        for (int m = 0; m < SPC; ++m) {
          uint32_t aw[4];
          if constexpr (FMT == FMT_F16) {
#pragma unroll
            for (int i = 0; i < 4; ++i) aw[i] = buf.k[st][j].w[i];
          } else if constexpr (FMT == FMT_INT8) {
            const uint32_t w0 = buf.k[st][j].w[2 * m], w1 = buf.k[st][j].w[2 * m + 1];
            aw[0] = perm(0u, w0, 0x0c010c00u);
            aw[1] = perm(0u, w0, 0x0c030c02u);
            aw[2] = perm(0u, w1, 0x0c010c00u);
            aw[3] = perm(0u, w1, 0x0c030c02u);
          } else {
            // bytes 0 and 2 (then 1 and 3, shifted down) already sit in the
            // low byte of each 16-bit half: one mask per pair of codes. High
            // nibbles stay in place (code * 16): the query slots they meet
            // carry 1/16, which saves their shift
            const uint32_t w = buf.k[st][j].w[m];
            const uint32_t w8 = w >> 8;
            aw[0] = w & 0x000F000Fu;  // elements 0, 4
            aw[1] = w8 & 0x000F000Fu; // elements 2, 6
            aw[2] = w & 0x00F000F0u;  // elements 1, 5 (x16)
            aw[3] = w8 & 0x00F000F0u; // elements 3, 7 (x16)
          }
          const half8_t av = __builtin_bit_cast(half8_t, (u32x4_t){aw[0], aw[1], aw[2], aw[3]});
          const int ks = j * SPC + m;
#pragma unroll
          for (int p = 0; p < PASSES; ++p)
#pragma unroll
            for (int h2 = 0; h2 < NQ; ++h2)
              cq[p] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, qb[p][h2][ks], cq[p], 0, 0, 0);
        }
      }
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int i = 4 * st + jj;
        float w = 0.f;
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
          if constexpr (QUANT) {
            const uint32_t mk = kmeta[p][i];
            w = fmaf(lo_f(mk), cq[p][jj], fmaf(hi_f(mk), qs[p], w));
          } else {
            w += cq[p][jj];
          }
        }
        w = sum_head_cols<G>(w); // the (group, hi/lo) columns of this head
        s[i] = (MASK && !ok[i]) ? -INFINITY : w;
      }
    }

    // ---- online softmax ----------------------------------------------------------
    const float tmax = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])),
                             fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
    m_true = fmaxf(m_true, tmax);
    if (__any(tmax > m_run + TAU_S)) { // wave-uniform, rare after the first tile
      float cand = fmaxf(m_run, tmax);
      for (int mask = G; mask < 16; mask <<= 1) cand = fmaxf(cand, __shfl_xor(cand, mask));
      cand = fmaxf(cand, xor16(cand));
      cand = fmaxf(cand, xor32(cand));
      // the running max moves on a grid of 2^-8 log2 units (rounded up), so
      // the offsets taken from it are exact: m_neg with WOFF, the rescale
      // factor and the wave's stored max. A rounding there would be one
      // factor shared by every weight of a rescale epoch or of a wave's
      // partial, which no later sum averages out.
      const float cl2 = ceilf(cand * (UNIT * 256.f)) * (1.f / 256.f);
      const float alpha = cand == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(fmaf(m_run, UNIT, -cl2));
      l_sum *= alpha;
#pragma unroll
      for (int p = 0; p < PASSES; ++p) zacc[p] *= alpha;
      // accumulator row 4r+i belongs to head (4r+i) mod G: take that
      // column's alpha; whole float4 accumulators are scaled, so each keeps
      // its registers (per-element products were moved back at every tile)
      float4_t a4;
#pragma unroll
      for (int i = 0; i < 4; ++i) a4[i] = __shfl(alpha, 16 * r + ((4 * r + i) & 15));
#pragma unroll
      for (int p = 0; p < PASSES; ++p)
#pragma unroll
        for (int e = 0; e < EV; ++e) acc[p][e] = acc[p][e] * a4;
      m_run = cl2 * (1.f / UNIT);
      m_neg = WOFF - cl2;
    }
    float pj[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) pj[i] = __builtin_amdgcn_exp2f(fmaf(s[i], UNIT, m_neg));
    l_sum += ((pj[0] + pj[1]) + (pj[2] + pj[3])) + ((pj[4] + pj[5]) + (pj[6] + pj[7]));

    // ---- weights: V scale folded in, binary16 hi/lo -------------------------------
    half8_t pa[PASSES][NQ];
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float w = pj[i];
        if constexpr (QUANT) {
          const uint32_t mv = vmeta[p][i];
          zacc[p] = fmaf(pj[i], fmaf(vmid<FMT>(), lo_f(mv), hi_f(mv)), zacc[p]);
          w *= lo_f(mv);
        }
        w = col_live ? w : 0.f;
        if constexpr (HL) {
          const _Float16 hi = (_Float16)w;
          // the lo half has its own accumulator rows, so it enters scaled by
          // 2^11 (it never exceeds the hi half, so this cannot overflow) and
          // stays out of the binary16 subnormal range; the rows are scaled
          // back where the wave's result is combined
          const _Float16 lo = (_Float16)((w - (float)hi) * LO_SCALE);
          pa[p][0][i] = col_lo ? lo : hi;
        } else {
          const _Float16 hi = (_Float16)w;
          const _Float16 lo = (_Float16)(w - (float)hi);
          pa[p][0][i] = hi;
          pa[p][NQ - 1][i] = lo;
        }
      }
    }

    // ---- values: B operand = 8 tokens of one dim, PV MFMA ----------------------------
#pragma unroll
    for (int e = 0; e < EV; ++e) {
      uint32_t bw[4];
#pragma unroll
      for (int q2 = 0; q2 < 4; ++q2) {
        const Raw<VB> &ta = buf.v[2 * q2], &tb = buf.v[2 * q2 + 1];
        if constexpr (FMT == FMT_F16) {
          bw[q2] = perm(tb.w[e / 2], ta.w[e / 2], (e & 1) ? 0x07060302u : 0x05040100u);
        } else if constexpr (FMT == FMT_INT8) {
          bw[q2] = centre_codes(perm(tb.w[e / 4], ta.w[e / 4], sel_pair(e & 3)), 128.f);
        } else {
          // odd dims (high nibbles) stay in place: code * 16, undone with
          // the code scale at the wave's result
          const uint32_t msk = (e & 1) ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
          const uint32_t na = ta.w[0] & msk;
          const uint32_t nb = tb.w[0] & msk;
          bw[q2] = centre_codes(perm(nb, na, sel_pair((e >> 1) & 3)), (e & 1) ? 8.f * INT4_HI : 8.f);
        }
      }
      const half8_t bv = __builtin_bit_cast(half8_t, (u32x4_t){bw[0], bw[1], bw[2], bw[3]});
#pragma unroll
      for (int p = 0; p < PASSES; ++p)
#pragma unroll
        for (int h2 = 0; h2 < NQ; ++h2)
          acc[p][e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[p][h2], bv, acc[p][e], 0, 0, 0);
    }
  };

  // ---- main loop: ring of DEPTH tiles ------------------------------------------
  // Every step issues the tile DEPTH-1 ahead and consumes one; tile k sits in
  // ring slot k % DEPTH. Whole rounds of DEPTH steps run with no exit inside a
  // round (the accumulators then stay in their registers across the loop;
  // early exits between steps made the compiler copy them at every tile),
  // then up to DEPTH-1 single steps. The last DEPTH-1 tiles are consumed
  // after the loop without issuing anything (the drain below), so no
  // zero-length loads are left in flight for the epilogue to wait on.
  // Masking: the drain holds the split's last tile, the only one that may end
  // past t1; split tile 0 starts before t0 only when t0 is not a multiple of
  // the tile, and then (the one case) every step of the loop is masked.
  // Inside a round the compiler schedules loads and compute freely (barriers
  // there cost 3 % on int4:32 and 6 % on long variable-length contiguous
  // batches); the single steps keep each step's loads ahead of its compute.
  // Binary16 rows with 4 waves and a ring of 2 take the per-step form instead
  // (an exit test before every step, each step masked only where its tile
  // crosses [t0, t1)): it compiles to 248 VGPRs against 255 plus 20 AGPRs for
  // whole rounds, which keeps two 4-wave workgroups per CU (2 % faster at GQA
  // 32/8 n32768 f16, 10 % on a batch of 16 sequences that needs several
  // rounds of workgroups); with 8 waves or a ring of 3 it measured slower
  // (median 1.3-1.8x over the f16 plans of the uniform sweep). (The per-step
  // loop is written inline below: wrapped in a lambda it compiled to 256
  // VGPRs plus 86 AGPRs.)
  constexpr bool PER_STEP = FMT == FMT_F16 && DEPTH == 2 && WPB == 4;
  int k = 0;
  auto stream = [&](auto mask_tag) __attribute__((always_inline)) {
    while (k + 2 * DEPTH - 1 <= nk) {
      static_for<DEPTH>([&](auto Ui) __attribute__((always_inline)) {
        constexpr int s = decltype(Ui)::value;
        issue(ring(std::integral_constant<int, (s + DEPTH - 1) % DEPTH>{}), k + DEPTH - 1);
        compute(ring(Ui), k, mask_tag);
        ++k;
      });
    }
    static_for<DEPTH - 1>([&](auto Ui) __attribute__((always_inline)) {
      constexpr int s = decltype(Ui)::value;
      if (k + DEPTH - 1 < nk) { // a prefix of the steps: once false, k stays put
        __builtin_amdgcn_sched_barrier(0);
        issue(ring(std::integral_constant<int, (s + DEPTH - 1) % DEPTH>{}), k + DEPTH - 1);
        __builtin_amdgcn_sched_barrier(0);
        compute(ring(Ui), k, mask_tag);
        ++k;
      }
    });
  };
  if constexpr (PER_STEP) {
    bool streaming = true;
    while (streaming) {
      static_for<DEPTH>([&](auto Ui) __attribute__((always_inline)) {
        constexpr int u = decltype(Ui)::value;
        if (!streaming) return;
        if (k + DEPTH - 1 >= nk) {
          streaming = false;
          return;
        }
        issue(ring(std::integral_constant<int, (u + DEPTH - 1) % DEPTH>{}), k + DEPTH - 1);
        const int tbase = (tile0 + tstep * (wave + nw * k)) * TT;
        if (tbase >= t0 && tbase + TT <= t1) compute(ring(Ui), k, std::false_type{});
        else compute(ring(Ui), k, std::true_type{});
        ++k;
      });
    }
  } else if (t0 % TT == 0) stream(std::false_type{});
  else stream(std::true_type{});
  // persistent step: thread 0 claims the workgroup's next item behind the
  // last tiles' loads, so the claim's round trip overlaps the drain
  unsigned claim = 0;
  if constexpr (QUEUE) {
    if (threadIdx.x == 0) claim = __hip_atomic_fetch_add(x.queue, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // drain: the tiles still in flight, masked (a full tile computes the same)
  for (int j = 0; j < DEPTH - 1; ++j, ++k) {
    if (k >= nk) break;
    static_for<DEPTH>([&](auto Ui) __attribute__((always_inline)) {
      if (k % DEPTH == decltype(Ui)::value) compute(ring(Ui), k, std::true_type{});
    });
  }

  // ---- wave result: per head (m_run, l, m_true) and O[head][D] ---------------
  l_sum += xor16(l_sum);
  l_sum += xor32(l_sum);
  m_true = fmaxf(m_true, xor16(m_true));
  m_true = fmaxf(m_true, xor32(m_true));
  float zrow[PASSES][4];
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    float z = zacc[p];
    z += xor16(z);
    z += xor32(z);
#pragma unroll
    for (int i = 0; i < 4; ++i) zrow[p][i] = __shfl(z, 16 * r + ((4 * r + i) & 15));
  }

  extern __shared__ __attribute__((aligned(16))) float smem[]; // 16 B: the fused merge reads float4
  // layout: sO[nw][G][D], sM[nw][G][3], then (HL_LDS) sL[nw][G][D]
  float *sO = smem;
  float *sM = smem + nw * G * D;
  float *sL = sM + nw * G * 3;
  if (r == 0 && c < G) {
    sM[(wave * G + c) * 3 + 0] = fmaf(m_run, UNIT, -WOFF);
    sM[(wave * G + c) * 3 + 1] = l_sum;
    sM[(wave * G + c) * 3 + 2] = m_true * UNIT;
  }
  const int gdim = (c * EV) / GRP; // group of this lane's V dims
  // With HL, accumulator rows 8-15 (lane-rows 2 and 3) hold the lo halves of
  // rows 0-7: they are stored to their own LDS rows (sL) and the combine adds
  // them, which keeps the cross-half sum off the VALU (the zero-point sum
  // enters once, with the hi half). Where sL would not fit beside sO, the
  // halves are summed with a lane swap instead.
  if constexpr (HL && !HL_LDS) {
#pragma unroll
    for (int e = 0; e < EV; ++e)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[0][e][i] = fmaf(xor32(acc[0][e][i]), LO_INV, acc[0][e][i]);
  }
#pragma unroll
  for (int p = 0; p < PASSES; ++p)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = p * 16 + 4 * r + i; // accumulator row
      const bool lo_half = HL && row >= 8;
      const int pr = HL ? (row & 7) : row; // its (group, head) pair
      const bool canon = HL ? (HL_LDS || !lo_half) && pr < COLS : (PASSES > 1 || pr < COLS);
      if (canon && (pr % COLS) / G == gdim) {
        float *dst = (lo_half ? sL : sO) + (wave * G + pr % G) * D + c * EV;
#pragma unroll
        for (int e = 0; e < EV; ++e)
          dst[e] = QUANT ? fmaf(acc[p][e][i], (lo_half ? CODE_UNIT * LO_INV : CODE_UNIT) * vdim_scale<FMT>(e),
                                lo_half ? 0.f : zrow[p][i])
                         : acc[p][e][i] * (lo_half ? LO_INV : 1.f);
      }
    }
  if constexpr (QUEUE) {
    if (threadIdx.x == 0) *s_next = claim;
  }
  __syncthreads();

  // every LDS read of an output element is issued before any is used: the
  // waves' (m_run, l, m_true) and partial outputs, then a branch-free
  // log-sum-exp over the waves (a wave with m_run = -inf saw no token and
  // contributes nothing; all -inf leaves L = O = 0)
  const int nthreads = nw * 64;
#pragma unroll
  for (int idx0 = 0; idx0 < G * D; idx0 += nthreads) {
    const int idx = idx0 + threadIdx.x;
    if (G * D % nthreads != 0 && idx >= G * D) break;
    const int hh = idx / D, col = idx % D;
    float mr[nw], lw[nw], mt[nw], ov[nw];
#pragma unroll
    for (int w2 = 0; w2 < nw; ++w2) {
      mr[w2] = sM[(w2 * G + hh) * 3 + 0];
      lw[w2] = sM[(w2 * G + hh) * 3 + 1];
      mt[w2] = sM[(w2 * G + hh) * 3 + 2];
      ov[w2] = sO[(w2 * G + hh) * D + col];
      if constexpr (HL_LDS) ov[w2] += sL[(w2 * G + hh) * D + col];
    }
    float M = -INFINITY;
#pragma unroll
    for (int w2 = 0; w2 < nw; ++w2) M = fmaxf(M, mt[w2]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < nw; ++w2) {
      const bool live = M != -INFINITY && mr[w2] != -INFINITY;
      const float wgt = live ? __builtin_amdgcn_exp2f(mr[w2] - M) : 0.f;
      L = live ? fmaf(lw[w2], wgt, L) : L;
      O = live ? fmaf(ov[w2], wgt, O) : O;
    }
    const int hq = G > 1 ? hkv * G + hh : hb;
    const long long head = (long long)b * a.H + hq;
    if (final_out) {
      const float res = L > 0.f ? O / L : 0.f;
      if (x.out16) x.out16[head * D + col] = (_Float16)res;
      else a.out[head * D + col] = res;
    } else {
      // agent-scope atomic stores: written through to the level every XCD
      // sees while the kernel still runs, so the fused step publishes them
      // without an L2 writeback, and in the two-launch step the writeback at
      // the kernel's end has no partials left to flush before the merge
      // (decode step, alternating rounds on two boxes: GQA 32/8 d128 int8
      // at 32k tokens 18.2 -> 17.6 us and 18.0 -> 17.9 us, int4 at 64k
      // 24.7 -> 24.2 us, a paged batch of 8 sequences 27.8 -> 28.0 us; the
      // split kernel alone 0.1 us longer)
      float *po = a.part_o + (head * a.splits + split) * D + col;
      float *pm = a.part_ml + (head * a.splits + split) * 2;
      __hip_atomic_store(po, O, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (col == 0) {
        __hip_atomic_store(pm, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(pm + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }

  // ---- fused merge: the last workgroup of a head group combines the splits ----
  // Every partial of this workgroup was written with an agent-scope atomic
  // store, which writes through to the device-coherent level; waiting for
  // the stores to complete orders them before this workgroup's arrival on
  // the counter, so no L2 writeback (the agent-scope release fence) is
  // needed. The workgroup that arrives last reads every partial of its head
  // group with device-coherent loads, which are served from that level too,
  // and resets the counter for the next call: every split has arrived by
  // then, so nothing touches the counter again in this call. The other
  // workgroups run the merge code dry (see merge_heads).
  if (!final_out && x.counters) {
    __shared__ unsigned s_last;
    unsigned *cnt = x.counters + ((long long)b * gy + hb) * KVF_COUNTER_STRIDE;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
      s_last = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (unsigned)(a.splits - 1);
    __syncthreads();
    const bool last = s_last != 0;
    // (the dry run pays only when every workgroup of the step is resident
    // at once, Ext::dry_merge; with more, and in the persistent loop, the
    // merge code is warm after the first round)
    if (last || (!QUEUE && x.dry_merge))
      merge_heads<D, G, WPB>(a, x, (long long)b * a.H + (G > 1 ? hkv * G : hb), !last);
    if (last && threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// The split kernel: a workgroup runs the one item its grid position names,
// (split, head group, sequence) = blockIdx on the 3-D grid, or the XCD-affine
// order of the fused step's 1-D grid (Ext::nx).
// Its first arguments repeat the fields the first loads wait for (the grid's
// XCD count, the sizes, the cache pointers, 14 dwords), ahead of Args and
// Ext: the kernel translation units are built with kernel-argument
// preloading of 14 dwords, so these arrive in SGPRs as the wave starts
// instead of through a load from the argument segment, and the rest of Args
// and Ext arrives while the first tiles' addresses are formed. The query
// pointer follows them. (Measured on MI355X, alternating builds, three
// rounds: the fused step 17.26-17.30 -> 17.01-17.07 us at GQA 32/8, d128,
// n32768, int8:64; config 3's fused step 28.18-28.19 -> 27.89-27.93 us; the
// two-launch steps within 0.05 us.)
template <int FMT, int D, int GQ, int G, int U, int ORD, bool PAGED, int WPB>
__global__ void __launch_bounds__(WPB * 64)
decode_partial(const int nx, const int n, const int splits, const int H, const int Hkv, const int B,
               const void *k, const void *v, const void *k_meta, const void *v_meta, const void *q,
               const Args args, const Ext ext, const int final_out) {
  Args a = args;
  a.n = n;
  a.splits = splits;
  a.H = H;
  a.Hkv = Hkv;
  a.B = B;
  a.k = static_cast<const unsigned char *>(k);
  a.v = static_cast<const unsigned char *>(v);
  a.k_meta = static_cast<const __half2 *>(k_meta);
  a.v_meta = static_cast<const __half2 *>(v_meta);
  a.q = static_cast<const float *>(q);
  Ext x = ext;
  x.nx = nx;
  const int gy = G > 1 ? a.Hkv : a.H; // head groups per sequence
  int split, hb, b;
  if (x.nx > 0) { // fused step on a 1-D grid: a head group's splits share an XCD
    const int m = a.B * gy / x.nx;
    const int q = (int)(blockIdx.x / x.nx);
    const int hg = (int)(blockIdx.x % x.nx) + x.nx * (q % m);
    split = q / m;
    b = hg / gy;
    hb = hg % gy;
  } else {
    split = blockIdx.x;
    hb = blockIdx.y;
    b = blockIdx.z;
  }
  decode_item<FMT, D, GQ, G, U, ORD, PAGED, WPB, false>(a, x, final_out, split, hb, b, nullptr);
}

// The persistent step's kernel (Ext::queue): a 1-D grid of at most as many
// workgroups as are resident at once works through a queue of the
// B * head groups * splits items, item i = split i % splits of head group
// (i / splits) % gy of sequence slot i / (splits * gy): slot-major, so with
// Ext::longest_first the longest sequences' items go first. Workgroup w
// starts on item w; each item claims the next (queue[0], counted from the
// grid size) while its last tiles are in flight, and a workgroup stops at a
// claim past the end: one atomic per item, not per tile. The last workgroup
// to stop (queue[KVF_COUNTER_STRIDE] counts them) returns both words to zero
// for the next call; every claim of every workgroup has returned before that
// workgroup is counted. A kernel of its own, because the loop around the
// item costs registers (spills in some variants) that the one-item kernel
// does not pay.
template <int FMT, int D, int GQ, int G, int U, int ORD, bool PAGED, int WPB>
__global__ void __launch_bounds__(WPB * 64)
decode_persistent(int, int, int, int, int, int, const void *, const void *, const void *, const void *,
                  const void *, const Args a, const Ext x, const int final_out) {
  const int gy = G > 1 ? a.Hkv : a.H;
  __shared__ unsigned s_next;
  const unsigned items = (unsigned)a.splits * (unsigned)gy * (unsigned)a.B;
  unsigned item = blockIdx.x;
  for (;;) {
    const int split = (int)(item % (unsigned)a.splits);
    const int rest = (int)(item / (unsigned)a.splits);
    decode_item<FMT, D, GQ, G, U, ORD, PAGED, WPB, true>(a, x, final_out, split, rest % gy, rest / gy,
                                                         &s_next);
    __syncthreads(); // the item's last LDS reads are done; s_next holds the claim
    item = gridDim.x + s_next;
    __syncthreads(); // every thread has read s_next before the next item rewrites it
    if (item >= items) break;
  }
  if (threadIdx.x == 0) {
    unsigned *done = x.queue + KVF_COUNTER_STRIDE;
    if (__hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1) {
      __hip_atomic_store(x.queue, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// Fused-step merge of the G heads [head0, head0 + G) by the last workgroup of
// their head group: the log-sum-exp recombination of decode_merge
// (runtime/kvf_kernels.cuh:288-306). One wave per head (a wave takes heads
// w, w + NW, ...), lane l owning output dims [l*EL, l*EL + EL). Per chunk of
// 32 splits a wave issues 33 loads: lane s < 32 loads split s's (max, sum)
// pair, and every lane loads its dims of the 32 split outputs, so a chunk is
// one memory round trip (the wave's outstanding-load counter holds 63). The
// chunk's max and weighted sum are wave reductions (DPP row rotations and
// lane swaps), and the split weights reach every lane through readlane into
// scalar registers, so the code is short and straight-line, which matters
// because it runs once per head group from a cold instruction cache. Empty
// splits (max -inf) and slots past the split count weigh nothing (every
// split writes its row on every call, an empty one zeros, so every row read
// is finite); more than 32 splits fold with a running max. Loads are
// device-coherent raw buffer loads through descriptors over the head's rows
// (a split past the end reads zero).
//
// Every workgroup of the head group runs this code once its arrival is
// counted: the last one on the partials, the others as a dry run (`dry`:
// zero-length descriptors, so no load reaches memory, one chunk of
// placeholder splits, and no stores), which brings the code into the XCD's
// L2 before the last workgroup fetches it. (Run cold, the code alone takes
// ~0.85 us of the ~1.8 us merge for GQA 32/8, d128, 32 splits.)
template <int D, int G, int NW>
__device__ __forceinline__ void merge_heads(const Args &a, const Ext &x, long long head0, bool dry) {
  constexpr int EL = D / 64; // output dims per lane
  constexpr int MCH = 32;    // splits per round trip
  constexpr int CPOL = CPOL_SC1;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int S = dry ? 1 : a.splits;
  for (int h = wave; h < G; h += NW) {
    const long long head = head0 + h;
    const __amdgpu_buffer_rsrc_t rml = rsrc(a.part_ml, head * S * 8, dry ? 0u : (uint32_t)(S * 8));
    const __amdgpu_buffer_rsrc_t ro = rsrc(a.part_o, head * S * D * 4, dry ? 0u : (uint32_t)(S * D * 4));
    float M = -INFINITY, L = 0.f, O[EL];
#pragma unroll
    for (int e = 0; e < EL; ++e) O[e] = 0.f;
    for (int s0 = 0; s0 < S; s0 += MCH) {
      const int sl = s0 + (lane & (MCH - 1));
      const i32x2_t p = __builtin_amdgcn_raw_buffer_load_b64(rml, sl * 8, 0, CPOL);
      Raw<EL * 4> o[MCH];
#pragma unroll
      for (int i = 0; i < MCH; ++i) bload<EL * 4, CPOL>(ro, ((s0 + i) * D + lane * EL) * 4, o[i]);
      // every load of the chunk goes out before any is used: one round trip
      __builtin_amdgcn_sched_barrier(0);
      // (elements go through plain ints: clang's __builtin_bit_cast of an
      // ext_vector element reads element 0 whichever element is named)
      const int pm = p.x, pl = p.y;
      const bool live = lane < MCH && sl < S;
      const float m = live ? (dry ? 0.f : __builtin_bit_cast(float, pm)) : -INFINITY;
      float Mc = fmaxf(M, m);
      Mc = fmaxf(Mc, ror16<1>(Mc));
      Mc = fmaxf(Mc, ror16<2>(Mc));
      Mc = fmaxf(Mc, ror16<4>(Mc));
      Mc = fmaxf(Mc, ror16<8>(Mc));
      Mc = fmaxf(Mc, xor16(Mc));
      Mc = fmaxf(Mc, xor32(Mc));
      Mc = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, Mc))); // equal in every lane
      // branch-free (a branch here let the compiler move the output loads
      // past the wait for the maxima: two round trips instead of one); while
      // every split so far is empty, all weights are 0 and L, O stay 0
      const float Mref = Mc == -INFINITY ? 0.f : Mc;
      const float alpha = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - Mref);
      const float w = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - Mref);
      float lw = live ? __builtin_bit_cast(float, pl) * w : 0.f;
      lw += ror16<1>(lw);
      lw += ror16<2>(lw);
      lw += ror16<4>(lw);
      lw += ror16<8>(lw);
      lw += xor16(lw);
      lw += xor32(lw);
      L = fmaf(L, alpha, lw);
#pragma unroll
      for (int e = 0; e < EL; ++e) O[e] *= alpha;
#pragma unroll
      for (int i = 0; i < MCH; ++i) {
        const float wi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), i));
#pragma unroll
        for (int e = 0; e < EL; ++e) O[e] = fmaf(__builtin_bit_cast(float, o[i].w[e]), wi, O[e]);
      }
      M = Mc;
    }
    if (dry) {
      asm volatile("" ::"v"(O[0]), "v"(L)); // keep the dry run's arithmetic
      continue;
    }
#pragma unroll
    for (int e = 0; e < EL; ++e) {
      const float res = L > 0.f ? O[e] / L : 0.f;
      if (x.out16) x.out16[head * D + lane * EL + e] = (_Float16)res;
      else a.out[head * D + lane * EL + e] = res;
    }
  }
}

// Stand-alone merge: one workgroup of D threads per (query head, sequence),
// thread d owning output dim d. Its arguments are six scalars (10 dwords)
// rather than Args, so all of them can arrive preloaded in SGPRs. It is the log-sum-exp recombination of
// runtime/kvf_kernels.cuh:288-306: M = max of the split maxima, empty splits
// (m = -inf) skipped, out = sum_s O_s 2^(m_s - M) / sum_s l_s 2^(m_s - M), 0
// when the sum is 0. Up to MERGE_CHUNK splits cost one memory round trip and
// need no LDS and no barrier (merge_chunks); beyond that, chunks are folded
// with a running max, and the launcher runs decode_merge_sliced below, which
// folds up to 8 chunks side by side. Loads go
// through buffer descriptors over the head's rows: a split past the end reads
// zero and is masked to m = -inf without a branch.
constexpr int MERGE_CHUNK = 32;

// Folds chunks c0, c0 + cstep, ... (MERGE_CHUNK splits each, below S) of one
// head into the running (M, L, O) of output dim d. Lane s of each wave (and
// s + 32) loads split s's (m, l) pair beside the thread's MERGE_CHUNK partial
// outputs, so a chunk is one memory round trip; the chunk maximum and the
// weighted sum of l are wave reductions (DPP row rotations, a lane swap), and
// each split's weight reaches every lane through readlane.
template <int D>
__device__ __forceinline__ void merge_chunks(__amdgpu_buffer_rsrc_t rml, __amdgpu_buffer_rsrc_t ro, int d, int S,
                                             int c0, int cstep, float &M, float &L, float &O) {
  static_assert(MERGE_CHUNK == 32, "a chunk is one pair per lane of half a wave");
  const int ls = threadIdx.x & 31;
  for (int s0 = c0 * MERGE_CHUNK; s0 < S; s0 += cstep * MERGE_CHUNK) {
    const i32x2_t p = __builtin_amdgcn_raw_buffer_load_b64(rml, (s0 + ls) * 8, 0, 0);
    float o[MERGE_CHUNK];
#pragma unroll
    for (int i = 0; i < MERGE_CHUNK; ++i)
      o[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ro, ((s0 + i) * D + d) * 4, 0, 0));
    // every load of the chunk goes out before any is used: one round trip
    // (left alone, the scheduler issues the output loads after the maxima
    // have arrived)
    __builtin_amdgcn_sched_barrier(0);
    const int pm = p.x, pl = p.y; // (element-wise, see merge_heads)
    // a split past the end reads zeros: m = -inf, l = 0
    const float m = s0 + ls < S ? __builtin_bit_cast(float, pm) : -INFINITY;
    float Mc = fmaxf(m, ror16<8>(m));
    Mc = fmaxf(Mc, ror16<4>(Mc));
    Mc = fmaxf(Mc, ror16<2>(Mc));
    Mc = fmaxf(Mc, ror16<1>(Mc));
    Mc = fmaxf(fmaxf(Mc, xor16(Mc)), M);
    // branch-free: while every split so far is empty, all weights are 0 and
    // L, O stay 0
    const float Mref = Mc == -INFINITY ? 0.f : Mc;
    const float alpha = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - Mref);
    const float w = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - Mref);
    float lw = __builtin_bit_cast(float, pl) * w;
    lw += ror16<8>(lw);
    lw += ror16<4>(lw);
    lw += ror16<2>(lw);
    lw += ror16<1>(lw);
    lw += xor16(lw);
    L = fmaf(L, alpha, lw);
    O *= alpha;
#pragma unroll
    for (int i = 0; i < MERGE_CHUNK; ++i)
      O = fmaf(o[i], __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), i)), O);
    M = Mc;
  }
}

template <int D>
__global__ void __launch_bounds__(D)
decode_merge(const float *part_o, const float *part_ml, float *out, _Float16 *out16, int H, int S) {
  const long long head = (long long)blockIdx.y * H + blockIdx.x;
  const int d = threadIdx.x;
  const __amdgpu_buffer_rsrc_t rml = rsrc(part_ml, head * S * 8, (uint32_t)(S * 8));
  const __amdgpu_buffer_rsrc_t ro = rsrc(part_o, head * S * D * 4, (uint32_t)(S * D * 4));
  float M = -INFINITY, L = 0.f, O = 0.f;
  merge_chunks<D>(rml, ro, d, S, 0, 1, M, L, O);
  const float res = L > 0.f ? O / L : 0.f;
  if (out16) out16[head * D + d] = (_Float16)res;
  else out[head * D + d] = res;
}

// The same merge for more than MERGE_CHUNK splits: NSL slices of D threads,
// slice k folding chunks k, k + NSL, ..., so up to NSL chunks are one memory
// round trip instead of one each; the slices' (M, L, O) then combine through
// LDS as the splits do (weights 2^(M_k - M), an empty slice weighing 0).
template <int D, int NSL>
__global__ void __launch_bounds__(NSL * D)
decode_merge_sliced(const float *part_o, const float *part_ml, float *out, _Float16 *out16, int H, int S) {
  __shared__ float sO[NSL][D];
  __shared__ float sM[NSL], sL[NSL];
  const long long head = (long long)blockIdx.y * H + blockIdx.x;
  const int d = threadIdx.x % D;
  const int sl = threadIdx.x / D;
  const __amdgpu_buffer_rsrc_t rml = rsrc(part_ml, head * S * 8, (uint32_t)(S * 8));
  const __amdgpu_buffer_rsrc_t ro = rsrc(part_o, head * S * D * 4, (uint32_t)(S * D * 4));
  float M = -INFINITY, L = 0.f, O = 0.f;
  merge_chunks<D>(rml, ro, d, S, sl, NSL, M, L, O);
  sO[sl][d] = O;
  if (d == 0) {
    sM[sl] = M;
    sL[sl] = L;
  }
  __syncthreads();
  if (sl == 0) {
    float Mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < NSL; ++k) Mx = fmaxf(Mx, sM[k]);
    float Lt = 0.f, Ot = 0.f;
#pragma unroll
    for (int k = 0; k < NSL; ++k) {
      const float w = sM[k] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sM[k] - Mx);
      Lt = fmaf(sL[k], w, Lt);
      Ot = fmaf(sO[k][d], w, Ot);
    }
    const float res = Lt > 0.f ? Ot / Lt : 0.f;
    if (out16) out16[head * D + d] = (_Float16)res;
    else out[head * D + d] = res;
  }
}

// Launches decode_merge<D>. Defined and instantiated (D = 64, 128) in
// kvf_merge.hip alone, which is built with its six arguments preloaded into
// SGPRs, so the merge starts its loads without a kernel-argument round trip.
template <int D> hipError_t launch_merge_kernel(const Args &a, const Ext &x, hipStream_t st);
extern template hipError_t launch_merge_kernel<64>(const Args &, const Ext &, hipStream_t);
extern template hipError_t launch_merge_kernel<128>(const Args &, const Ext &, hipStream_t);

// Compute units and XCDs of the current device, queried once per device.
struct DevInfo {
  int cus = 0, nx = 1;
};
inline hipError_t dev_info(DevInfo &out) {
  static std::mutex mu;
  static std::map<int, DevInfo> cache;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(dev);
  if (it == cache.end()) {
    DevInfo d;
    e = hipDeviceGetAttribute(&d.cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    if (hipDeviceGetAttribute(&d.nx, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || d.nx < 1) d.nx = 1;
    it = cache.emplace(dev, d).first;
  }
  out = it->second;
  return hipSuccess;
}

template <int FMT, int D, int GQ, int G, int U, int ORD, bool PAGED>
hipError_t launch_group(const Args &a, const Ext &x, const Launch &l, hipStream_t st) {
  const int gy = G > 1 ? a.Hkv : a.H;
  dim3 grid(a.splits, gy, a.B);
  const dim3 block(a.warps * 64);
  const int final_out = (a.splits == 1 && !l.partial_only) ? 1 : 0;
  const bool fused = x.counters && !final_out && !l.partial_only;
  Ext xk = x;
  if (!fused) xk.counters = nullptr;
  xk.nx = 0;
  if (fused) {
    // one launch: when the head groups divide evenly over the device's XCDs,
    // a 1-D grid places every split of a head group on one XCD
    DevInfo di;
    const hipError_t e = dev_info(di);
    if (e != hipSuccess) return e;
    const int nhg = a.B * gy;
    // (head-major rows only: with token-major rows every KV head sits at one
    // byte offset of each token's row, and one head per XCD made a paged
    // token-major batch of 8 sequences take 38 us fused against 28 us on the
    // (splits, heads, B) grid)
    // (uniform lengths only: the 1-D order runs split by split over all head
    // groups, which undoes longest-first and lets short sequences' splits
    // crowd out the long ones; a batch of 16 sequences with log-uniform
    // lengths up to 128k took 145 us fused on it against 94 us on the
    // (splits, heads, B) grid)
    // (a 1-D grid holds at most 2^32 - 1 work-items: larger steps keep the
    // 3-D grid)
    if (ORD == ORD_HEAD && !x.seq_lens && di.nx > 1 && nhg % di.nx == 0 &&
        (long long)a.splits * nhg * block.x <= 0xffffffffLL) {
      xk.nx = di.nx;
      grid = dim3((unsigned)(a.splits * nhg));
    }
  }
  const size_t lds = combine_lds<FMT, D, GQ, G>(a.warps);
  auto kernel = a.warps == 4 ? &decode_partial<FMT, D, GQ, G, U, ORD, PAGED, 4>
                             : &decode_partial<FMT, D, GQ, G, U, ORD, PAGED, 8>;
  // workgroups of a kernel resident per CU (occupancy API), looked up once per
  // kernel; slot 0/1: the one-item kernel with 4/8 waves, 2/3: the persistent one
  auto resident_per_cu = [&](const void *k, int slot, int &out) -> hipError_t {
    static std::atomic<int> cache[4] = {-1, -1, -1, -1};
    out = cache[slot].load(std::memory_order_relaxed);
    if (out < 0) {
      const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&out, k, (int)block.x, lds);
      if (e != hipSuccess) return e;
      cache[slot].store(out, std::memory_order_relaxed);
    }
    out = std::max(1, out);
    return hipSuccess;
  };
  const int wslot = a.warps == 4 ? 0 : 1;
  DevInfo di;
  if (fused || x.queue) {
    const hipError_t e = dev_info(di);
    if (e != hipSuccess) return e;
  }
  int per_cu = 0; // one-item kernel
  if (fused || x.queue) {
    const hipError_t e = resident_per_cu(reinterpret_cast<const void *>(kernel), wslot, per_cu);
    if (e != hipSuccess) return e;
  }
  if (fused) {
    // the dry merge warms the merge code only where every workgroup of the
    // step is resident at once (one round)
    xk.dry_merge = (long long)grid.x * grid.y * grid.z <= (long long)per_cu * di.cus;
  }
  if (x.queue) {
    // persistent step: a 1-D grid of at most the persistent kernel's
    // workgroups resident at once (more could not start before others
    // finish, so they would only add claims), capped by Ext::slots. Without
    // a cap, a step whose items all fit in the one-item kernel's resident
    // grid has nothing to queue, and the static grid above runs instead.
    // (built for unroll 2 only, which keeps the library's build time near
    // what it was without the persistent kernels)
    if (l.partial_only || U != 2) return hipErrorInvalidValue;
    auto pk = a.warps == 4 ? &decode_persistent<FMT, D, GQ, G, 2, ORD, PAGED, 4>
                           : &decode_persistent<FMT, D, GQ, G, 2, ORD, PAGED, 8>;
    const long long items = (long long)a.splits * gy * a.B;
    if (items > 0x7fffffffLL) return hipErrorInvalidValue;
    int pers_per_cu = 0;
    const hipError_t e = resident_per_cu(reinterpret_cast<const void *>(pk), 2 + wslot, pers_per_cu);
    if (e != hipSuccess) return e;
    long long wgs = std::min<long long>(items, (long long)pers_per_cu * di.cus);
    if (x.slots > 0) wgs = std::min<long long>(wgs, x.slots);
    const bool queue = x.slots > 0 ? wgs < items : items > (long long)per_cu * di.cus;
    if (queue) {
      kernel = pk;
      grid = dim3((unsigned)wgs);
      xk.nx = 0;
    } else {
      xk.queue = nullptr;
    }
  }
  // the split kernel's leading scalars (see decode_partial; the persistent
  // kernel takes the same list and reads Args)
  const void *kp = a.k, *vp = a.v, *kmp = a.k_meta, *vmp = a.v_meta, *qp = a.q;
  if (l.ev_start || l.ev_stop)
    hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, st, l.ev_start, l.ev_stop, 0, xk.nx, a.n, a.splits,
                          a.H, a.Hkv, a.B, kp, vp, kmp, vmp, qp, a, xk, final_out);
  else
    hipLaunchKernelGGL(kernel, grid, block, lds, st, xk.nx, a.n, a.splits, a.H, a.Hkv, a.B, kp, vp, kmp, vmp, qp,
                       a, xk, final_out);
  if (!final_out && !l.partial_only && !fused) return launch_merge_kernel<D>(a, x, st);
  return hipGetLastError();
}

// Checks what the kernels assume about Args before anything is launched.
inline bool args_ok(const Args &a, int fmt, int D, int G, bool paged) {
  if (a.warps != 4 && a.warps != 8) return false;
  if (a.B < 1 || a.H < 1 || a.Hkv < 1 || a.n < 0 || a.splits < 1) return false;
  if (a.B > 65535 || a.H > 65535 || a.splits > 65535) return false;
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
hipError_t launch_ext(const Args &a, const Ext &x, const Launch &l, hipStream_t st) {
  if (!args_ok(a, FMT, D, G, PAGED)) return hipErrorInvalidValue;
  if (a.n == 0) return hipErrorInvalidValue;
  if constexpr (FMT == FMT_F16) {
    return launch_group<FMT, D, 0, G, U, ORD, PAGED>(a, x, l, st);
  } else {
    switch (a.group_shift) {
    case 5: return launch_group<FMT, D, 32, G, U, ORD, PAGED>(a, x, l, st);
    case 6: return launch_group<FMT, D, 64, G, U, ORD, PAGED>(a, x, l, st);
    default:
      if constexpr (D >= 128) return launch_group<FMT, D, 128, G, U, ORD, PAGED>(a, x, l, st);
      return hipErrorInvalidValue;
    }
  }
}

} // namespace gfx950

// The registry-facing template (runtime/kvf_kernels.cuh:309-320 signature).
template <int FMT, int D, int G, int U, int ORD, bool PAGED>
hipError_t launch(const Args &a, hipStream_t st) {
  return gfx950::launch_ext<FMT, D, G, U, ORD, PAGED>(a, gfx950::Ext{}, gfx950::Launch{}, st);
}

} // namespace kvf
