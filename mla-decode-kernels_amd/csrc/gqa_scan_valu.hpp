// The VALU scan of one (request, kv-head) segment by a workgroup of P waves:
// tile loads, QK^T / online softmax / PV per tile, and the fixed-order merges
// of row and wave states. Shared by the split-rule kernels
// (gqa_decode_split.hip) and the token-balanced persistent kernel
// (gqa_decode_balanced.hip); everything here is force-inlined into them.
//
// A wave's 64 lanes form 4 DPP rows of 16 lanes; a row reads one 256-byte K
// (or V) head row with 16-byte loads, so one load instruction covers 4 tokens
// and a 16-token tile is 4 K loads + 4 V loads per lane. Per tile: QK^T with
// v_dot2c_f32_bf16 on the packed bf16 q and K words, a 4-step DPP row
// reduction, then one online-softmax update per (row, head) for the whole tile
// (max over its 4 tokens, one rescale of l and acc) in base-2 units, and PV as
// fp32 FMAs. The next tile's loads are issued before the current tile is
// consumed.
#pragma once

#include <type_traits>

#include "gqa_device.hpp"
#include "gqa_scan.hpp"

namespace gqa {

constexpr int kTile = 16;        // tokens per wave per tile
constexpr int kChunkAlign = 32;  // split lengths are multiples of this (both split-rule kernels)
constexpr int kLoads = 4;        // 16-byte K loads (and V loads) per lane per tile

// Launch shapes. A workgroup holds P waves that share one kv-head, take its
// 16-token tiles round-robin and merge their states through LDS. Measured on
// MI355X: the stream runs fastest with about one wave per SIMD resident (4 per
// CU), each keeping one tile in flight while it consumes the previous one;
// more resident waves or deeper prefetch only add queueing. P = 4 waves per
// kv-head keeps a workgroup's reads adjacent and the merge in LDS.
constexpr int kWavesPerHead = 4;  // P: waves sharing a kv-head (all scan kernels)
constexpr int kScanDepth = 2;     // register tiles in flight per wave

struct TileRegs {
  uint4 k[kLoads];
  uint4 v[kLoads];
};

// Online-softmax state of GH q-heads in one lane: m and l per head (identical
// across the 16 lanes of a DPP row), acc over the lane's 8 dims.
template <int GH>
struct WaveState {
  float m[GH], l[GH], acc[GH][8];
};

template <int GH>
__device__ __forceinline__ void init_state(WaveState<GH>& st) {
#pragma unroll
  for (int j = 0; j < GH; ++j) {
    st.m[j] = kNegInf;
    st.l[j] = 0.f;
#pragma unroll
    for (int d = 0; d < 8; ++d) st.acc[j][d] = 0.f;
  }
}

// q rows of heads h0 .. h0 + nh - 1 of request b: lane dims [8c, 8c + 8);
// heads past nh are zero (their results are never written).
template <int GH>
__device__ __forceinline__ void load_q(const ScanArgs& a, int b, int h0, int nh, int c,
                                       uint4 (&qf)[GH]) {
#pragma unroll
  for (int j = 0; j < GH; ++j) {
    qf[j] = make_uint4(0, 0, 0, 0);
    if (j < nh)
      qf[j] = *reinterpret_cast<const uint4*>(a.q + ((size_t)b * a.Hq + h0 + j) * kHeadDim + 8 * c);
  }
}

// The tile work of one wave on kv-head hkv of the request whose block table
// row is bt: issue() loads the K and V rows of the 16-token tile starting at
// token ts, consume() folds a loaded tile into the wave's state. Tokens at or
// past `end` (the end of the segment being scanned) are never read: their
// loads read the tile's first token instead (always valid), so no load touches
// an unallocated block or a tail slot, and consume<true> masks their scores.
template <int GH, bool kBlockUniform>
struct ValuTiles {
  const ScanArgs& a;
  const int* bt;
  // The block table is read-only for the whole launch: reading it through the
  // constant address space lets the uniform block-id loads stay scalar even
  // in kernels that store to global memory between segments.
  const __attribute__((address_space(4))) int* btc;
  int hkv, r, c, bs;
  uint32_t row_elems, row_bytes;  // elements (bytes) between slots
  const uint16_t* kbase;
  const uint16_t* vbase;
  // Per-lane byte offsets of the tile's K/V loads from its first slot's
  // kv-head row: load j reads token 4j + r, dims [8c, 8c + 8). A block's
  // bytes fit 32 bits (checked at launch), so each load is a uniform 64-bit
  // base plus one of these fixed 32-bit lane offsets.
  uint32_t loff[kLoads];

  __device__ __forceinline__ ValuTiles(const ScanArgs& a_, const int* bt_, int hkv_, int r_, int c_)
      : a(a_),
        bt(bt_),
        btc((const __attribute__((address_space(4))) int*)bt_),
        hkv(hkv_),
        r(r_),
        c(c_),
        bs(a_.block_size),
        row_elems((uint32_t)a_.Hkv * kHeadDim),
        row_bytes((uint32_t)a_.Hkv * kHeadDim * 2u),
        kbase(a_.k_cache + (size_t)hkv_ * kHeadDim + 8 * c_),
        vbase(a_.v_cache + (size_t)hkv_ * kHeadDim + 8 * c_) {
#pragma unroll
    for (int j = 0; j < kLoads; ++j) loff[j] = (uint32_t)(4 * j + r) * row_bytes + 16u * c;
  }

  __device__ __forceinline__ void issue(int ts, int end, TileRegs& t) const {
    if constexpr (kBlockUniform) {
      // The 16 tokens of the tile share one block: scalar block-id load and a
      // uniform base at the tile's first slot.
      const uint32_t lb = fastdiv((uint32_t)ts, a.bs_div);
      const uint32_t slot0 = (uint32_t)ts - lb * (uint32_t)bs;
      const size_t base = ((size_t)btc[lb] * bs + slot0) * row_bytes + (size_t)hkv * (kHeadDim * 2);
      const auto kr = kv_rsrc(reinterpret_cast<const char*>(a.k_cache) + base);
      const auto vr = kv_rsrc(reinterpret_cast<const char*>(a.v_cache) + base);
      // No branch between full and partial tiles here: a uniform branch around
      // the loads made the waits after it conservative (measured: 15% slower).
#pragma unroll
      for (int j = 0; j < kLoads; ++j) {
        const uint32_t off = ts + 4 * j + r < end ? loff[j] : 16u * c;
        t.k[j] = load_kv(kr, off);
        t.v[j] = load_kv(vr, off);
      }
    } else {
#pragma unroll
      for (int j = 0; j < kLoads; ++j) {
        int tok = ts + 4 * j + r;
        tok = tok < end ? tok : ts;
        const uint32_t lb = fastdiv((uint32_t)tok, a.bs_div);
        const int slot = tok - (int)lb * bs;
        const size_t off = ((size_t)bt[lb] * bs + slot) * row_elems;
        t.k[j] = load_kv(kbase + off);
        t.v[j] = load_kv(vbase + off);
      }
    }
  }

  // Fold the tile starting at ts into st. kMasked: the tile may reach past
  // end; scores of tokens at or past end become -inf.
  template <bool kMasked>
  __device__ __forceinline__ void consume(int ts, int end, const uint4 (&qf)[GH], const TileRegs& t,
                                          WaveState<GH>& st) const {
    float s[kLoads][GH];  // raw scores q.k, then probabilities
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
#pragma unroll
      for (int h = 0; h < GH; ++h) {
        float d = dot2_bf16(qf[h].x, t.k[j].x, 0.f);
        d = dot2_bf16(qf[h].y, t.k[j].y, d);
        d = dot2_bf16(qf[h].z, t.k[j].z, d);
        d = dot2_bf16(qf[h].w, t.k[j].w, d);
        d = row16_sum(d);
        if constexpr (kMasked) d = ts + 4 * j + r < end ? d : kNegInf;
        s[j][h] = d;
      }
    }
    // New running max of each head in scaled base-2 units. The state is
    // rescaled only when some head's max moved in some lane of the wave (a
    // wave-uniform branch; after a segment's first tiles it is rare), and the
    // factor of an unmoved head is exactly 1, so skipping changes no bit.
    float mn[GH];
    bool moved = false;
#pragma unroll
    for (int h = 0; h < GH; ++h) {
      const float mt = fmaxf(fmaxf(s[0][h], s[1][h]), fmaxf(s[2][h], s[3][h]));
      mn[h] = fmaxf(st.m[h], mt * a.scale_log2e);
      moved |= mn[h] != st.m[h];
    }
    if (__builtin_amdgcn_ballot_w64(moved)) {
#pragma unroll
      for (int h = 0; h < GH; ++h) {
        // m = -inf (no valid token yet) gives a factor of 0 on l = acc = 0.
        const float al = mn[h] == st.m[h] ? 1.f : exp2_fast(st.m[h] - mn[h]);
        st.m[h] = mn[h];
        st.l[h] *= al;
#pragma unroll
        for (int d = 0; d < 8; ++d) st.acc[h][d] *= al;
      }
    }
#pragma unroll
    for (int h = 0; h < GH; ++h) {
      // p = 2^(s * scale * log2(e) - m). Unmasked tiles make m finite; a row
      // of a masked tile may have no valid token yet (m = -inf, scores -inf),
      // and exp2(-inf) = 0 then needs a finite offset.
      const float nm = kMasked && st.m[h] == kNegInf ? 0.f : -st.m[h];
#pragma unroll
      for (int j = 0; j < kLoads; ++j) s[j][h] = exp2_fast(fmaf(s[j][h], a.scale_log2e, nm));
      st.l[h] += (s[0][h] + s[1][h]) + (s[2][h] + s[3][h]);
    }
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
      const float vf[8] = {bf16_lo(t.v[j].x), bf16_hi(t.v[j].x), bf16_lo(t.v[j].y),
                           bf16_hi(t.v[j].y), bf16_lo(t.v[j].z), bf16_hi(t.v[j].z),
                           bf16_lo(t.v[j].w), bf16_hi(t.v[j].w)};
#pragma unroll
      for (int h = 0; h < GH; ++h)
#pragma unroll
        for (int d = 0; d < 8; ++d) st.acc[h][d] = fmaf(s[j][h], vf[d], st.acc[h][d]);
    }
  }
};

// Scan tokens [seg_start, seg_end) of kv-head hkv of the request whose block
// table row is bt: wave ph of the P takes tiles ph, ph + P, ... of the range and
// folds them into st. DEPTH register tiles are in flight; the steady-state
// loop issues tile k + DEPTH - 1 before consuming tile k and has no branch, so
// the wait before each consume covers only the tile being consumed.
// kPinIssue puts a scheduling barrier after each tile's loads: without it the
// compiler may sink a tile's loads below the previous tile's arithmetic, so
// that tile is consumed right after its loads are issued. Measured on MI355X:
// pinning speeds the token-balanced kernel up ~5% (ragged B=128 batch) and is
// neutral to 1% slower for the split-rule kernel, whose default schedule
// already overlaps.
template <int GH, int P, int DEPTH, bool kBlockUniform, bool kPinIssue = false>
__device__ __forceinline__ void scan_segment(const ScanArgs& a, const int* bt, int hkv,
                                             const uint4 (&qf)[GH], int seg_start, int seg_end,
                                             int ph, int r, int c, WaveState<GH>& st) {
  // The steady-state loop leaves each wave's last tile (the only one that can
  // reach past seg_end) to the masked tail only with two or more tiles in
  // flight.
  static_assert(DEPTH >= 2, "scan_segment needs at least two tiles in flight");
  const int ntiles = (seg_end - seg_start + kTile - 1) / kTile;
  const int my_tiles = ntiles > ph ? (ntiles - ph + P - 1) / P : 0;
  const ValuTiles<GH, kBlockUniform> tiles(a, bt, hkv, r, c);

  auto tile_start = [&](int k) { return seg_start + kTile * (ph + P * k); };
  auto issue = [&](int k, TileRegs& t) { tiles.issue(tile_start(k), seg_end, t); };
  auto consume = [&](int k, const TileRegs& t, auto masked) {
    tiles.template consume<decltype(masked)::value>(tile_start(k), seg_end, qf, t, st);
  };
  constexpr std::true_type kTail{};
  constexpr std::false_type kFull{};

  if (my_tiles > 0) {
    TileRegs t[DEPTH];
#pragma unroll
    for (int i = 0; i < DEPTH - 1; ++i)
      if (i < my_tiles) issue(i, t[i]);
    int k = 0;
    for (; k + 2 * DEPTH - 2 < my_tiles; k += DEPTH) {
#pragma unroll
      for (int i = 0; i < DEPTH; ++i) {
        issue(k + i + DEPTH - 1, t[(i + DEPTH - 1) % DEPTH]);
        if constexpr (kPinIssue) __builtin_amdgcn_sched_barrier(0);
        consume(k + i, t[i], kFull);
      }
    }
#pragma unroll
    for (int i = 0; i < DEPTH; ++i) {
      if (k + i < my_tiles) {
        if (k + i + DEPTH - 1 < my_tiles) issue(k + i + DEPTH - 1, t[(i + DEPTH - 1) % DEPTH]);
        if constexpr (kPinIssue) __builtin_amdgcn_sched_barrier(0);
        consume(k + i, t[i], kTail);
      }
    }
#pragma unroll
    for (int i = 0; i < DEPTH - 1; ++i) {
      // At most 2*DEPTH - 2 tiles remain after the loop; the block above
      // consumed DEPTH of them.
      if (k + DEPTH + i < my_tiles) {
        if (k + DEPTH + i + DEPTH - 1 < my_tiles)
          issue(k + DEPTH + i + DEPTH - 1, t[(i + 2 * DEPTH - 1) % DEPTH]);
        consume(k + DEPTH + i, t[(DEPTH + i) % DEPTH], kTail);
      }
    }
  }
}

// One wave scans tokens [rs, re) of kv-head hkv in consecutive 16-token tiles,
// where rs is the start of a split and the splits are tps tiles long (tps
// even: split lengths are multiples of kChunkAlign tokens), and calls
// flush(st) at the end of each split it scans -- the last one ends at re --
// which must store the state and re-initialise it. Two tiles are in flight
// across split boundaries as well, so the loads of a split's first tiles are
// issued while the previous split's last tile is folded: a wave's splits
// stream as one segment. Split boundaries fall after odd-numbered tiles only,
// so the boundary test runs once per pair of tiles.
template <int GH, bool kBlockUniform, class Flush>
__device__ __forceinline__ void scan_split_range(const ScanArgs& a, const int* bt, int hkv,
                                                 const uint4 (&qf)[GH], int rs, int re, int tps,
                                                 int r, int c, WaveState<GH>& st, Flush&& flush) {
  const int ntiles = (re - rs + kTile - 1) / kTile;
  if (ntiles <= 0) return;
  const ValuTiles<GH, kBlockUniform> tiles(a, bt, hkv, r, c);
  TileRegs t0, t1;
  tiles.issue(rs, re, t0);
  int k = 0, left = tps;
  for (; k + 2 < ntiles; k += 2) {  // tiles k and k + 1 are whole and not the last
    const int ts = rs + kTile * k;
    tiles.issue(ts + kTile, re, t1);
    tiles.template consume<false>(ts, re, qf, t0, st);
    tiles.issue(ts + 2 * kTile, re, t0);
    tiles.template consume<false>(ts + kTile, re, qf, t1, st);
    left -= 2;
    if (left == 0) {
      flush(st);
      left = tps;
    }
  }
  const int ts = rs + kTile * k;
  if (k + 1 < ntiles) {
    tiles.issue(ts + kTile, re, t1);
    tiles.template consume<true>(ts, re, qf, t0, st);
    tiles.template consume<true>(ts + kTile, re, qf, t1, st);
  } else {
    tiles.template consume<true>(ts, re, qf, t0, st);
  }
  flush(st);
}

// Merge the 4 row states of the wave in place (every row ends with the same
// totals): Mw / Lw get the wave's max and sum, st.acc the rescaled sums.
template <int GH>
__device__ __forceinline__ void merge_rows(WaveState<GH>& st, float (&Mw)[GH], float (&Lw)[GH]) {
#pragma unroll
  for (int h = 0; h < GH; ++h) {
    const float mr = st.m[h];
    const float M = xor32_max(xor16_max(mr));
    const float f = mr == M ? 1.f : exp2_fast(mr - (M == kNegInf ? 0.f : M));
    const float lr = xor32_sum(xor16_sum(st.l[h] * f));
#pragma unroll
    for (int d = 0; d < 8; ++d) st.acc[h][d] = xor32_sum(xor16_sum(st.acc[h][d] * f));
    Mw[h] = M;
    Lw[h] = lr;
  }
}

// LDS staging of the P wave states of a workgroup (acc first: its rows take
// 16-byte stores).
template <int GH, int P>
struct WaveMergeLds {
  float acc[P][GH][kHeadDim];
  float m[P][GH];
  float l[P][GH];
};

// Wave ph stores its merged state (row 0 holds it after merge_rows).
template <int GH, int P>
__device__ __forceinline__ void stage_wave_state(WaveMergeLds<GH, P>& lds, int ph, int lane,
                                                 int r, int c, const WaveState<GH>& st,
                                                 const float (&Mw)[GH], const float (&Lw)[GH]) {
#pragma unroll
  for (int h = 0; h < GH; ++h) {
    if (r == 0) {
      float4* dst = reinterpret_cast<float4*>(&lds.acc[ph][h][8 * c]);
      dst[0] = make_float4(st.acc[h][0], st.acc[h][1], st.acc[h][2], st.acc[h][3]);
      dst[1] = make_float4(st.acc[h][4], st.acc[h][5], st.acc[h][6], st.acc[h][7]);
    }
    if (lane == 0) {
      lds.m[ph][h] = Mw[h];
      lds.l[ph][h] = Lw[h];
    }
  }
}

// Combine the P staged wave states of head h at dim d in wave order:
// M = max, L = sum of rescaled l, A = sum of rescaled acc. The factor of a wave
// holding the max is exactly 1. M is in base-2 units.
template <int GH, int P>
__device__ __forceinline__ void merge_wave_states(const WaveMergeLds<GH, P>& lds, int h, int d,
                                                  float& M, float& L, float& A) {
  M = lds.m[0][h];
#pragma unroll
  for (int w = 1; w < P; ++w) M = fmaxf(M, lds.m[w][h]);
  const float Ms = M == kNegInf ? 0.f : M;
#pragma unroll
  for (int w = 0; w < P; ++w) {
    const float mw = lds.m[w][h];
    const float f = mw == M ? 1.f : exp2_fast(mw - Ms);
    if (w == 0) {
      L = lds.l[0][h] * f;
      A = lds.acc[0][h][d] * f;
    } else {
      L = fmaf(lds.l[w][h], f, L);
      A = fmaf(lds.acc[w][h][d], f, A);
    }
  }
}

// q-heads served per wave of the VALU scan: the whole group (at most 4 here),
// rounded up to a power of two; extra heads carry q = 0 and are not written.
inline int heads_per_wave(int G) { return G <= 1 ? 1 : G <= 2 ? 2 : 4; }

}  // namespace gqa
