// MLA absorbed-path paged decode for gfx950 (the reference's roadmap item K2,
// README.md:405-408): every query row (s_q x h_q of a request) attends over
// one shared latent cache of 576-dim rows; values are the rows' first 512
// dims. Semantics and layouts: include/mla_decode.h.
//
// Work decomposition. A workgroup of 4 waves (one per SIMD) owns 128 query
// rows (a row group) of one request and a range of its tokens; each wave owns
// 32 rows as two 16-row MFMA column blocks. All rows share the cache rows, so
// each 32-token tile (36 KiB) is read from HBM once per workgroup: the waves
// copy it cooperatively, HBM -> LDS (global_load_lds_dwordx4, no registers),
// into a ring of kDepth slots with kDepth - 1 tiles in flight, and every wave
// computes from LDS. Two launches share this tile walk (mla_piece):
//   fixed splits  grid (row groups, B, num_splits), split s of each request;
//   balanced      one workgroup per CU and row group, each taking an equal
//                 share of the batch's request-ordered tiles (a plan kernel
//                 computes the tile prefix sums on the device), walked piece
//                 by piece; requests cut between shares are merged after.
//
// LDS tile layout: 4 row blocks of 8 tokens, each 9 column blocks of 1 KiB
// (8 rows x 128 bytes = 64 dims) plus 16 bytes, so that consecutive row
// blocks start 16 bytes apart modulo the 256-byte bank cycle; within a column
// block, row r sits at 128 r and its 16-byte chunk c at position
// c ^ chunk_swz(r). Each copy instruction fills one column block: 8 lanes per
// row read that row's 128 contiguous bytes from HBM (a copy of 16 rows x 64
// bytes per instruction streamed at ~4.5 TB/s, 8 x 128 bytes at ~6.2 TB/s,
// measured on MI355X), and the swizzle only permutes lanes within a row.
// Both operand reads below are free of bank conflicts in this layout (the
// QK ds_read_b128 phases of 16 lanes and the PV ds_read_b64_tr_b16 groups),
// and both address as a per-lane base plus a per-step immediate.
//
//   QK^T   S^T[16 tok x 16 rows] = K[tok x 576] . Q^T[576 x 16 rows]: 18
//          MFMAs per token group and row block; A from LDS (lane: token j,
//          dims 32 kk + 8 g; shared by both row blocks), B = Q^T in registers
//          (lane: row j, dims 32 kk + 8 g).
//   softmax on the C layout (lane: row j, tokens 4 g + e), base 2, fp32,
//          against a per-row reference max fixed at the row's first live
//          tile (see kRefSlack); P rounded to bf16, l sums the rounded values.
//   PV     O[16 rows x 512] += P[rows x 32 tok] . V[32 tok x 512]: 32
//          v_mfma_f32_16x16x32_bf16 per row block (k-slot 8g+e -> token
//          4g+e, 8g+4+e -> token 16+4g+e); B read from the same LDS tile with
//          ds_read_b64_tr_b16 (lane x of a 16-lane group supplies token
//          4g + x/4, dims 16nb + 4(x%4) .. +4; the transpose hands lane x the
//          four tokens of dim 16nb + x).
//
// Splits and shares cut requests at multiples of 32 tokens; the merges fold
// the pieces in order (log-sum-exp), so results are bitwise reproducible.
#include "gqa_device.hpp"
#include "gqa_launch.hpp"
#include "mla_decode.h"

#include <algorithm>

namespace mla {

using gqa::exp2_fast;
using gqa::f32_to_bf16_bits;
using gqa::FastDiv;
using gqa::kLn2;
using gqa::kLog2e;
using gqa::kNegInf;

constexpr int kD = MLA_DECODE_HEAD_DIM;     // 576
constexpr int kDV = MLA_DECODE_HEAD_DIM_V;  // 512
constexpr int kKSteps = kD / 32;            // 18 QK k-steps
constexpr int kTile = 32;                   // tokens per tile
constexpr int kWaves = 4;
constexpr int kRowsPerWave = 32;
constexpr int kRowsPerGroup = kWaves * kRowsPerWave;  // 128
constexpr int kTileBlocks = 2 * kKSteps;              // 36 blocks of 1 KiB
constexpr int kColBlocks = kD / 64;                   // 9 per row block of 8 tokens
constexpr int kRowBlockBytes = kColBlocks * 1024 + 16;
constexpr int kTileBytes = 4 * kRowBlockBytes;
constexpr int kStageLoads = kTileBlocks / kWaves;     // 9 per wave per tile
// Tiles in the LDS ring: while a tile is consumed, the next kDepth - 1 are in
// flight from HBM (about 100 KiB per CU, enough to cover the latency at this
// CU's share of the bandwidth).
constexpr int kDepth = 4;
constexpr int kNB = kDV / 16;                         // 32 PV column blocks
static_assert(kTileBlocks % kWaves == 0, "staging blocks must split evenly");
static_assert(kTileBlocks == 4 * kColBlocks, "a tile is 4 row blocks of 9 column blocks");

// Position XOR of row r's 16-byte chunks in a column block (a table found by
// an exhaustive bank-conflict check of both operand reads over this layout).
__device__ __forceinline__ int chunk_swz(int r) { return (int)((0x46226400u >> (4 * r)) & 7u); }

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4_t;

struct MlaArgs {
  const uint16_t* q;
  const uint16_t* kv;
  const int* block_table;
  const int* seq_lens;
  uint16_t* out;
  float* lse;
  float* ws_acc;  // [B, R, ns, 512]
  float* ws_m;    // [B, R, ns] natural-log units
  float* ws_l;
  const uint64_t* pre;  // balanced launch: tile prefix sums [B + 1]
  const int* first;     // balanced launch: each share's first request
  int B, s_q, h_q, R, block_size, max_blocks, num_splits, causal, nshare;
  FastDiv bs_div;
  float scale_log2e;
};

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4& u) {
  return __builtin_bit_cast(bf16x8_t, u);
}

// One row block's running state; lane (j, g): m and lsum of row j (lsum over
// this lane's token slots only), o[nb][e] = O[row 4g + e][dim 16 nb + j].
struct RowState {
  float m, lsum;
  f32x4_t o[kNB];
};

// A row's probabilities are taken relative to a reference max that is set by
// the first tile holding a live key of the row and then kept: rescaling the
// 32 x 512 fp32 accumulators (all 256 accumulation registers of the lane) on
// every new max would cost more than the tile's matrix work, and any
// conditional update of them inside the tile loop makes the compiler copy them
// on every tile. Probabilities stay below 2^kRefSlack; if a later tile beats a
// row's reference by more, the workgroup runs its split a second time against
// the rows' true maxima (the values are exact either way; only that split's
// time doubles).
constexpr float kRefSlack = 32.f;
// LDS operand reads run this many MFMA steps ahead of their use: QK k-steps
// (4 MFMAs each) and PV column blocks (2 MFMAs each).
constexpr int kQKAhead = 2;
constexpr int kPVAhead = 4;

// Direct HBM -> LDS copies of 16 bytes per lane (global_load_lds_dwordx4):
// lane x's bytes land at LDS byte address lds + 16 x; lds must be
// wave-uniform. They are issued through inline assembly so that the compiler
// does not tie its LDS reads of the other ring slots to these loads'
// completion (it would wait for every load in flight before each read);
// completion is awaited explicitly with s_waitcnt vmcnt before the barrier
// that publishes a tile. The first form addresses base + voff (a uniform
// 64-bit base, a 32-bit per-lane offset); the second a per-lane address.
// On gfx9-family GPUs an LDS-DMA instruction needs one wait state after an
// SALU write of M0; the compiler inserts it for its own LDS-DMA code but does
// not look inside inline assembly, hence the s_nop (measured cost: up to ~3 %
// on the matrix-bound s_q = 2 workloads).
// M0 is a register the compiler reserves (hipcc notes the clobber as such and
// will not restore it): these kernels rely on the compiler emitting no M0 use
// of its own, which tests/test_mla_codegen.py checks on the generated code,
// together with the spill-free and wait-free tile loops.
__device__ __forceinline__ void load_to_lds(const uint16_t* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt"
               :
               : "v"(voff), "s"(base), "s"(lds)
               : "memory", "m0");
}
__device__ __forceinline__ void load_to_lds(const uint16_t* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
               :
               : "v"(src), "s"(lds)
               : "memory", "m0");
}

// Waits until at most kInFlight of this wave's direct loads are outstanding
// (they complete in issue order), then joins the workgroup barrier; LDS reads
// and writes are not moved across it.
template <int kInFlight>
__device__ __forceinline__ void publish_barrier() {
  static_assert(kInFlight >= 0 && kInFlight < 64, "vmcnt holds 6 bits");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(kInFlight) : "memory");
}

// Max over lanes l, l ^ 16, l ^ 32 and l ^ 48, the four lanes that hold one
// row in the MFMA C layout: v_permlane16_swap (v_permlane32_swap) with both
// operands x hands every lane x of itself and of its xor-16 (xor-32) partner,
// in VALU registers (no LDS round trip). The two results are copied out of the
// builtin's vector as plain integers before any bit cast: this clang lowers
// __builtin_bit_cast of an element (b[1]) as a read of element 0, which drops
// the partner's value and with it the max.
__device__ __forceinline__ float row_max(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const uint32_t a0 = a[0], a1 = a[1];
  const float y = fmaxf(__uint_as_float(a0), __uint_as_float(a1));
  const uint32_t v = __float_as_uint(y);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  const uint32_t b0 = b[0], b1 = b[1];
  return fmaxf(__uint_as_float(b0), __uint_as_float(b1));
}

// Where a piece's results go: normalised rows to out and lse (direct), or
// unnormalised states, row r of the piece's request at index
// st_base + r * st_stride of ws_acc (x 512), ws_m and ws_l.
struct PieceOut {
  bool direct;
  size_t st_base;
  int st_stride;
};

// The workgroup's 128 query rows (row group rg) of request b against tokens
// [seg_start, seg_end) of the request's S live tokens. Every wave of the
// workgroup calls it with the same arguments (its barriers are workgroup-wide).
template <bool kBlockUniform>
__device__ __forceinline__ void mla_piece(const MlaArgs& a, uint8_t (*tiles)[kTileBytes],
                                          int* restart_vote, int b, int rg, int S, int seg_start,
                                          int seg_end, PieceOut po) {
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  // Copies: lane x fills row cr = x / 8 of a column block, position x % 8,
  // from that row's chunk cc = (x % 8) ^ chunk_swz(cr).
  const int cr = lane >> 3, cc = (lane & 7) ^ chunk_swz(lane >> 3);
  // Tile-relative LDS offsets of this lane's operands (plus a per-step
  // immediate): QK A operand of token group tg, k-step parity par (token
  // 16 tg + j, chunk 4 par + g of column block kk / 2), and PV B operand of
  // column-block quarter q = nb % 4 (tokens 4 g + j / 4 (+16), dims
  // 16 nb + 4 (j % 4) .. +4: chunk 2 q + (j % 4) / 2, half j % 2).
  // (Token group 1 is two row blocks on: an immediate.)
  uint32_t qoff[2], voff4[4];
#pragma unroll
  for (int par = 0; par < 2; ++par)
    qoff[par] = (uint32_t)((j >> 3) * kRowBlockBytes + (j & 7) * 128 +
                           16 * ((4 * par + g) ^ chunk_swz(j & 7)));
  {
    const int vr = 4 * (g & 1) + (j >> 2);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      voff4[q] = (uint32_t)((g >> 1) * kRowBlockBytes + vr * 128 +
                            16 * ((2 * q + ((j & 3) >> 1)) ^ chunk_swz(vr)) + 8 * (j & 1));
  }
  // Waves whose rows all lie past R compute on zero queries (their results are
  // not stored): a wave-dependent branch around the tile work would make the
  // compiler copy the accumulators on every tile.
  const int row0 = rg * kRowsPerGroup + w * kRowsPerWave;
  const int ntiles = (seg_end - seg_start + kTile - 1) / kTile;

  // Q^T as the B operand, all 18 k-steps in registers (lane: row j, dims
  // 32 kk + 8 g); and each lane's key limit for its row j.
  uint4 qf[2][kKSteps];
  int lim[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int r = row0 + 16 * rb + j;
    const bool live = r < a.R;
    const uint16_t* qrow = a.q + ((size_t)b * a.R + (live ? r : 0)) * kD + 8 * g;
#pragma unroll
    for (int kk = 0; kk < kKSteps; ++kk)
      qf[rb][kk] = live ? *reinterpret_cast<const uint4*>(qrow + 32 * kk) : make_uint4(0, 0, 0, 0);
    const int qi = live ? r / a.h_q : 0;
    lim[rb] = min(seg_end, a.causal ? S - (a.s_q - 1 - qi) : S);
  }
  // Let the Q loads land here: a wait left to their first use would sit inside
  // the tile loop, where it would also wait for every tile copy in flight.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)

  const int* bt = a.block_table + (size_t)b * a.max_blocks;
  // The table is read-only for the launch; through the constant address space
  // the uniform block-id loads become scalar loads.
  const __attribute__((address_space(4))) int* btc =
      (const __attribute__((address_space(4))) int*)bt;
  const int bs = a.block_size;
  typedef __attribute__((address_space(3))) uint8_t lds_u8;
  const uint32_t tiles_lds = (uint32_t)(uintptr_t)(lds_u8*)&tiles[0][0];

  // Staging of tile k into ring slot k % kDepth: wave w copies column blocks
  // blk = w + 4 i (i < 9): row block rb8 = blk / 9 (tokens 8 rb8 .. +8),
  // column block cb = blk % 9 (dims 64 cb .. +64). A lane's row is
  // 8 rb8 + cr; tokens at or past seg_end read the tile's first token instead
  // (masked later), so nothing outside the request's live cache rows is
  // touched. Block ids come from scalar loads, which keeps the vector memory
  // counter for the copies alone.
  // The refill copies of the block-uniform path are issued two per QK^T
  // k-step rather than in one burst after the barrier (a burst queues behind
  // the other waves' copies and holds the wave); Plan carries what they need,
  // and the block id is loaded one iteration ahead, before the barrier, so
  // that its scalar-load latency overlaps the wait for the landing tile.
  // (Plan holds only wave-uniform values: a lane's source offset is its row
  // offset, or its chunk of the tile's first token for rows past seg_end.)
  struct Plan {
    const uint16_t* base;
    int nvalid;
    uint32_t slot;
  };
  const uint32_t lane_row_off = (uint32_t)(cr * kD + 8 * cc) * 2u, lane_first_off = 16u * cc;
  auto block_id = [&](int k) -> int {
    return btc[gqa::fastdiv((uint32_t)(seg_start + kTile * k), a.bs_div)];
  };
  // The LDS address of column block blk of the slot at `slot`.
  auto block_lds = [&](uint32_t slot, int blk) -> uint32_t {
    const int rb8 = blk / kColBlocks, cb = blk - rb8 * kColBlocks;
    return slot + (uint32_t)(rb8 * kRowBlockBytes + cb * 1024);
  };
  auto prep = [&](int k, int id) -> Plan {
    const int ts = seg_start + kTile * k;
    Plan p;
    p.slot = tiles_lds + (uint32_t)(k % kDepth) * kTileBytes;
    const uint32_t lb = gqa::fastdiv((uint32_t)ts, a.bs_div);
    const size_t row0 = (size_t)id * bs + (ts - (int)lb * bs);
    p.base = a.kv + row0 * kD;
    p.nvalid = seg_end - ts;
    return p;
  };
  auto issue = [&](const Plan& p, int i) {
    const int blk = w + kWaves * i;
    const int rb8 = blk / kColBlocks, cb = blk - rb8 * kColBlocks;
    const uint32_t voff = 8 * rb8 + cr < p.nvalid ? lane_row_off + (uint32_t)(8 * rb8 * kD * 2)
                                                  : lane_first_off;
    load_to_lds(p.base + 64 * cb, voff, __builtin_amdgcn_readfirstlane(block_lds(p.slot, blk)));
  };
  auto stage = [&](int k) {
    const int ts = seg_start + kTile * k;
    const uint32_t slot = tiles_lds + (uint32_t)(k % kDepth) * kTileBytes;
    if constexpr (kBlockUniform) {
      // 32 tokens from a 32-aligned start share one block: a uniform base row.
      const Plan p = prep(k, btc[gqa::fastdiv((uint32_t)ts, a.bs_div)]);
#pragma unroll
      for (int i = 0; i < kStageLoads; ++i) issue(p, i);
    } else {
      // The tile's tokens span blocks lb_lo .. lb_hi: fetch their ids with
      // uniform loads and let each lane take its own rows (one per row block).
      const int t_hi = min(ts + kTile, seg_end) - 1;
      const int lb_lo = (int)gqa::fastdiv((uint32_t)ts, a.bs_div);
      const int lb_hi = (int)gqa::fastdiv((uint32_t)t_hi, a.bs_div);
      int tok[4], lbl[4];
      size_t row[4] = {0, 0, 0, 0};
#pragma unroll
      for (int rb8 = 0; rb8 < 4; ++rb8) {
        tok[rb8] = ts + 8 * rb8 + cr < seg_end ? 8 * rb8 + cr : 0;
        lbl[rb8] = (int)gqa::fastdiv((uint32_t)(ts + tok[rb8]), a.bs_div);
      }
      for (int q = lb_lo; q <= lb_hi; ++q) {
        const size_t id = (size_t)btc[q];
#pragma unroll
        for (int rb8 = 0; rb8 < 4; ++rb8) row[rb8] = lbl[rb8] == q ? id : row[rb8];
      }
      const uint16_t* src[4];
#pragma unroll
      for (int rb8 = 0; rb8 < 4; ++rb8)
        src[rb8] = a.kv + (row[rb8] * bs + (ts + tok[rb8] - lbl[rb8] * bs)) * kD + 8 * cc;
#pragma unroll
      for (int i = 0; i < kStageLoads; ++i) {
        const int blk = w + kWaves * i;
        const int rb8 = blk / kColBlocks, cb = blk - rb8 * kColBlocks;
        load_to_lds(src[rb8] + 64 * cb, __builtin_amdgcn_readfirstlane(block_lds(slot, blk)));
      }
    }
  };

  f32x4_t o[2][kNB];
  float lsum[2];
  float mref[2] = {kNegInf, kNegInf};  // row j's reference max (log2 units)
  float mtrue[2] = {kNegInf, kNegInf};  // row j's max over the split so far
  bool beaten = false;                  // some row's max beat its reference

  // One pass over the split's tiles, accumulating o and lsum against mref.
  auto pass = [&]() {
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      lsum[rb] = 0.f;
#pragma unroll
      for (int nb = 0; nb < kNB; ++nb) o[rb][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    int id_next = 0;
    if constexpr (kBlockUniform) {
      if (kDepth - 1 < ntiles) id_next = block_id(kDepth - 1);
    }
    // Prologue: tiles 0 .. kDepth - 2 in flight; tile 0 published.
    for (int k = 0; k < kDepth - 1 && k < ntiles; ++k) stage(k);
    if (ntiles >= kDepth - 1)
      publish_barrier<kStageLoads * (kDepth - 2)>();
    else
      publish_barrier<0>();
    for (int k = 0; k < ntiles; ++k) {
      // Refill the slot consumed in the previous iteration (every wave has
      // passed the barrier that ended it).
      const bool refill = k + kDepth - 1 < ntiles;
      Plan pl;
      if constexpr (kBlockUniform) {
        if (refill) pl = prep(k + kDepth - 1, id_next);
      } else {
        if (refill) stage(k + kDepth - 1);
      }
      const uint8_t* T = tiles[k % kDepth];
      const int ts = seg_start + kTile * k;

      // QK^T: c[rb][tg][e] = score of token 16 tg + 4 g + e for row j of block rb.
      // Operand reads run kQKAhead k-steps ahead of their MFMAs (the
      // scheduling barriers keep the compiler from sinking them to their use).
      auto read_k = [&](int kk, int tg) -> uint4 {
        return *reinterpret_cast<const uint4*>(T + qoff[kk & 1] + 2 * kRowBlockBytes * tg +
                                               1024 * (kk >> 1));
      };
      f32x4_t c[2][2];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int tg = 0; tg < 2; ++tg) c[rb][tg] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      uint4 kr[kQKAhead + 1][2];
#pragma unroll
      for (int kk = 0; kk < kQKAhead; ++kk)
#pragma unroll
        for (int x = 0; x < 2; ++x) kr[kk][x] = read_k(kk, x);
#pragma unroll
      for (int kk = 0; kk < kKSteps; ++kk) {
        if (kk + kQKAhead < kKSteps) {
          const int sl = (kk + kQKAhead) % (kQKAhead + 1);
#pragma unroll
          for (int x = 0; x < 2; ++x) kr[sl][x] = read_k(kk + kQKAhead, x);
        }
        if constexpr (kBlockUniform) {
          if ((kk & 1) == 0 && refill) issue(pl, kk >> 1);  // copies 0..8 of the refill
        }
        __builtin_amdgcn_sched_barrier(0);
        const int sl = kk % (kQKAhead + 1);
#pragma unroll
        for (int tg = 0; tg < 2; ++tg)
#pragma unroll
          for (int rb = 0; rb < 2; ++rb)
            c[rb][tg] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                as_bf16x8(kr[sl][tg]), as_bf16x8(qf[rb][kk]), c[rb][tg], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }

      // V operands for PV, read kPVAhead column blocks ahead of their MFMAs;
      // the first ones are issued before the softmax. Lane (j, g) supplies
      // token 4g + j/4 (and 16 more: two row blocks on), dims 16nb + 4(j%4)
      // .. +4; the transposing read hands lane x the four tokens of dim
      // 16nb + x.
      auto read_v = [&](int nb) -> bf16x8_t {
        const uint32_t off = voff4[nb & 3] + 1024u * (uint32_t)(nb >> 2);
        const bf16x4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)(T + off));
        const bf16x4_t v1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (lds_bf16x4_t*)(T + off + 2 * kRowBlockBytes));
        return bf16x8_t{v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
      };
      bf16x8_t vr[kPVAhead + 1];
#pragma unroll
      for (int nb = 0; nb < kPVAhead; ++nb) vr[nb] = read_v(nb);
      __builtin_amdgcn_sched_barrier(0);

      // Probabilities against the reference max, rounded to bf16 (l sums the
      // rounded values).
      uint32_t pw[2][4];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        float sc[2][4];
        float mx = kNegInf;
#pragma unroll
        for (int tg = 0; tg < 2; ++tg)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const bool valid = ts + 16 * tg + 4 * g + e < lim[rb];
            sc[tg][e] = valid ? c[rb][tg][e] * a.scale_log2e : kNegInf;
            mx = fmaxf(mx, sc[tg][e]);
          }
        // mx is this lane's max (its 8 tokens of row j). The row's first live
        // tile sets the reference (nothing is accumulated before it, so
        // nothing needs rescaling); the row's four lanes agree on it.
        mref[rb] = mref[rb] == kNegInf ? row_max(mx) : mref[rb];
        beaten |= mx > mref[rb] + kRefSlack;
        mtrue[rb] = fmaxf(mtrue[rb], mx);  // lane-local until a second pass
        const float base = mref[rb] == kNegInf ? 0.f : mref[rb];
        float psum = 0.f;
#pragma unroll
        for (int tg = 0; tg < 2; ++tg)
#pragma unroll
          for (int e = 0; e < 4; e += 2) {
            const gqa::bf16x2_t pb = __builtin_convertvector(
                (float __attribute__((ext_vector_type(2)))){exp2_fast(sc[tg][e] - base),
                                                            exp2_fast(sc[tg][e + 1] - base)},
                gqa::bf16x2_t);
            const uint32_t wd = __builtin_bit_cast(uint32_t, pb);
            pw[rb][2 * tg + e / 2] = wd;
            psum += gqa::bf16_lo(wd) + gqa::bf16_hi(wd);
          }
        lsum[rb] += psum;
      }

      // PV: o[rb][nb] += P[16 rows x 32 tok] . V[32 tok x dims 16nb .. +16].
#pragma unroll
      for (int nb = 0; nb < kNB; ++nb) {
        if (nb + kPVAhead < kNB) vr[(nb + kPVAhead) % (kPVAhead + 1)] = read_v(nb + kPVAhead);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
          const bf16x8_t pa =
              as_bf16x8(make_uint4(pw[rb][0], pw[rb][1], pw[rb][2], pw[rb][3]));
          o[rb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, vr[nb % (kPVAhead + 1)],
                                                              o[rb][nb], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      // The block id the next iteration's copies need, loaded here so that
      // its latency overlaps the wait below.
      if constexpr (kBlockUniform) {
        if (k + kDepth < ntiles) id_next = block_id(k + kDepth);
      }
      // Tile k + 1 must have landed; the later ones stay in flight.
      if (refill)
        publish_barrier<kStageLoads * (kDepth - 2)>();
      else
        publish_barrier<0>();
    }
  };

  pass();
  // A row whose max beat its reference by more than kRefSlack has overflowed
  // or lost precision: the workgroup (which stages tiles together) runs the
  // split again with every row's reference at its true max (probabilities
  // <= 1, so a second pass always suffices). The ballot is taken with the
  // whole wave active (each lane holds its own rows' and tokens' flag); only
  // the store is lane 0's.
  const bool wave_beaten = __builtin_amdgcn_ballot_w64(beaten) != 0;
  if (lane == 0) restart_vote[w] = wave_beaten;
  __syncthreads();
  if (restart_vote[0] | restart_vote[1] | restart_vote[2] | restart_vote[3]) {
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      mref[rb] = row_max(mtrue[rb]);
    }
    pass();
  }

  // Final (m, l) of the rows this lane's o entries hold: rows 4g + e.
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    float L = lsum[rb] + __shfl_xor(lsum[rb], 16, 64);
    L += __shfl_xor(L, 32, 64);
    float Me[4], Le[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      Me[e] = __shfl(mref[rb], 4 * g + e, 64);
      Le[e] = __shfl(L, 4 * g + e, 64);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = row0 + 16 * rb + 4 * g + e;
      if (row >= a.R) continue;
      const size_t br = (size_t)b * a.R + row;
      if (po.direct) {
        const float inv = Le[e] > 0.f ? 1.f / Le[e] : 0.f;
#pragma unroll
        for (int nb = 0; nb < kNB; ++nb)
          a.out[br * kDV + 16 * nb + j] = (uint16_t)f32_to_bf16_bits(o[rb][nb][e] * inv);
        if (a.lse && j == 0) {
          const int qi = row / a.h_q, h = row - qi * a.h_q;
          a.lse[((size_t)b * a.h_q + h) * a.s_q + qi] =
              Le[e] > 0.f ? Me[e] * kLn2 + logf(Le[e]) : kNegInf;
        }
      } else {
        const size_t sx = po.st_base + (size_t)row * po.st_stride;
#pragma unroll
        for (int nb = 0; nb < kNB; ++nb) a.ws_acc[sx * kDV + 16 * nb + j] = o[rb][nb][e];
        if (j == 0) {
          a.ws_m[sx] = Le[e] > 0.f ? Me[e] * kLn2 : kNegInf;  // natural-log units
          a.ws_l[sx] = Le[e];
        }
      }
    }
  }
}

// Fixed splits: workgroup (rg, b, split) takes split `split` of request b,
// cut at multiples of 32 tokens.
template <bool kBlockUniform>
__global__ __launch_bounds__(256, 1) void mla_decode_kernel(const MlaArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t tiles[kDepth][kTileBytes];
  __shared__ int restart_vote[kWaves];
  const int b = blockIdx.y, split = blockIdx.z;
  const int s_cap = a.max_blocks * a.block_size;
  const int S = min(max(a.seq_lens[b], 0), s_cap);
  const int ns = a.num_splits;
  const int chunk = ((S + ns - 1) / ns + (kTile - 1)) & ~(kTile - 1);
  const int seg_start = min(split * chunk, S);
  const int seg_end = min(S, seg_start + chunk);
  PieceOut po;
  po.direct = ns == 1;
  po.st_base = (size_t)b * a.R * ns + split;
  po.st_stride = ns;
  mla_piece<kBlockUniform>(a, tiles, restart_vote, b, blockIdx.x, S, seg_start, seg_end, po);
}

// Log-sum-exp fold of `count` states of one (request, query row), in order,
// into out and lse: one wave per row, lane i owns dims 8i .. 8i + 8. index(i)
// is the state index of the i-th; states with m = -inf (no key) add nothing.
template <typename IndexFn>
__device__ __forceinline__ void merge_row(const MlaArgs& a, size_t br, int count, IndexFn index) {
  constexpr int kBatch = 8;
  const int lane = threadIdx.x & 63;
  float mloc = kNegInf;
  for (int i = lane; i < count; i += 64) mloc = fmaxf(mloc, a.ws_m[index(i)]);
  const float M = gqa::wave_max(mloc);
  float L = 0.f, A[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) A[d] = 0.f;
  if (M != kNegInf) {
    for (int i0 = 0; i0 < count; i0 += kBatch) {
      float mi[kBatch], li[kBatch];
      float4 a0[kBatch], a1[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const size_t sx = index(min(i0 + k, count - 1));  // past the end: valid, not folded
        mi[k] = a.ws_m[sx];
        li[k] = a.ws_l[sx];
        const float4* src = reinterpret_cast<const float4*>(a.ws_acc + sx * kDV + 8 * lane);
        a0[k] = src[0];
        a1[k] = src[1];
      }
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        if (i0 + k >= count) break;
        // Exactly 1 for the state holding the max; 0 for empty states.
        const float f = mi[k] == M ? 1.f : exp2_fast((mi[k] - M) * kLog2e);
        const float av[8] = {a0[k].x, a0[k].y, a0[k].z, a0[k].w, a1[k].x, a1[k].y, a1[k].z, a1[k].w};
        L = fmaf(li[k], f, L);
#pragma unroll
        for (int d = 0; d < 8; ++d) A[d] = fmaf(av[d], f, A[d]);
      }
    }
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  uint32_t wv[4];
#pragma unroll
  for (int d = 0; d < 4; ++d)
    wv[d] = f32_to_bf16_bits(A[2 * d] * inv) | (f32_to_bf16_bits(A[2 * d + 1] * inv) << 16);
  *reinterpret_cast<uint4*>(a.out + br * kDV + 8 * lane) = make_uint4(wv[0], wv[1], wv[2], wv[3]);
  if (a.lse && lane == 0) {
    const int b = (int)(br / a.R), row = (int)(br - (size_t)b * a.R);
    const int qi = row / a.h_q, h = row - qi * a.h_q;
    a.lse[((size_t)b * a.h_q + h) * a.s_q + qi] = L > 0.f ? M + logf(L) : kNegInf;
  }
}

// Fixed splits: the num_splits states of each row, in split order.
__global__ __launch_bounds__(256) void mla_decode_merge_kernel(const MlaArgs a) {
  const size_t br = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (br >= (size_t)a.B * a.R) return;
  const int ns = a.num_splits;
  merge_row(a, br, ns, [&](int i) { return br * ns + i; });
}

// ---------------------------------------------------------------------------
// Token-balanced launch. The work is the concatenation, in request order, of
// every request's 32-token tiles: T = sum_b ceil(S_b / 32). Share w of
// nshare (one workgroup per row group) takes tiles [w T / n, (w + 1) T / n)
// -- equal to within one tile, whatever the lengths -- and walks them piece
// by piece (a piece: the share's tiles of one request). A piece that is a
// whole request is normalised into out directly; only a share's first and
// last piece can be partial, and their states go to the share's two slots
// (2w, 2w + 1). The merge then folds each cut request's pieces in share order,
// so results are bitwise reproducible for a given nshare. With fewer tiles
// than shares, only the first T shares take work (one tile each), so every
// working share is non-empty.

// Share w's first tile.
__device__ __forceinline__ uint64_t share_start(uint64_t T, int w, int n) {
  return (uint64_t)w * T / (uint64_t)n;
}

// Tile prefix sums pre[b] = sum_{b' < b} ceil(S_b' / 32) (b = 0..B, S clamped
// to the block table), the working share count pre[B + 1] = min(nshare, T),
// and each working share's first request (the first b with pre[b + 1] > its
// first tile); one workgroup.
__global__ __launch_bounds__(256) void mla_plan_kernel(const MlaArgs a, uint64_t* pre, int* first) {
  __shared__ uint64_t part[256];
  const int tid = threadIdx.x;
  const int per = (a.B + 255) / 256;
  const int b0 = min(tid * per, a.B), b1 = min(b0 + per, a.B);
  const int s_cap = a.max_blocks * a.block_size;
  auto tiles_of = [&](int b) -> uint64_t {
    const int S = min(max(a.seq_lens[b], 0), s_cap);
    return (uint64_t)((S + kTile - 1) / kTile);
  };
  uint64_t sum = 0;
  for (int b = b0; b < b1; ++b) sum += tiles_of(b);
  part[tid] = sum;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {  // inclusive scan of the 256 partial sums
    const uint64_t v = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  uint64_t run = part[tid] - sum;
  for (int b = b0; b < b1; ++b) {
    pre[b] = run;
    run += tiles_of(b);
  }
  const uint64_t T = part[255];
  const int n = (int)(T < (uint64_t)a.nshare ? T : (uint64_t)a.nshare);
  if (tid == 0) {
    pre[a.B] = T;
    pre[a.B + 1] = (uint64_t)n;
  }
  __syncthreads();  // the prefix sums, written by all threads, are read below
  for (int w = tid; w < n; w += 256) {
    const uint64_t t = share_start(T, w, n);
    int lo = 0, hi = a.B - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (pre[mid + 1] > t) hi = mid; else lo = mid + 1;
    }
    first[w] = lo;
  }
}

// Workgroup (w, rg): share w of row group rg.
template <bool kBlockUniform>
__global__ __launch_bounds__(256, 1) void mla_decode_balanced_kernel(const MlaArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t tiles[kDepth][kTileBytes];
  __shared__ int restart_vote[kWaves];
  const int w = blockIdx.x, rg = blockIdx.y;
  const int s_cap = a.max_blocks * a.block_size;
  const uint64_t T = a.pre[a.B];
  const int n = (int)a.pre[a.B + 1];
  if (w >= n) return;
  const uint64_t t0 = share_start(T, w, n), t_end = share_start(T, w + 1, n);
  int b = a.first[w];
  for (uint64_t t = t0; t < t_end; ++b) {
    const uint64_t p0 = a.pre[b], p1 = a.pre[b + 1];
    if (p1 <= t) continue;  // a request with no tiles
    const uint64_t t1 = p1 < t_end ? p1 : t_end;
    const int S = min(max(a.seq_lens[b], 0), s_cap);
    PieceOut po;
    po.direct = t == p0 && t1 == p1;
    po.st_base = (size_t)(2 * w + (t == t0 ? 0 : 1)) * a.R;
    po.st_stride = 1;
    mla_piece<kBlockUniform>(a, tiles, restart_vote, b, rg, S, (int)(t - p0) * kTile,
                             min(S, (int)(t1 - p0) * kTile), po);
    t = t1;
  }
}

// Rows of requests cut by share boundaries: fold their pieces in share order
// (shares with no tiles hold no piece). Requests with no tiles get out = 0 and
// lse = -inf; whole pieces were written by the decode kernel.
__global__ __launch_bounds__(256) void mla_decode_balanced_merge_kernel(const MlaArgs a) {
  const size_t br = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (br >= (size_t)a.B * a.R) return;
  const int b = (int)(br / a.R), row = (int)(br - (size_t)b * a.R);
  const uint64_t p0 = a.pre[b], p1 = a.pre[b + 1], T = a.pre[a.B];
  const int n = (int)a.pre[a.B + 1];
  if (p1 == p0) {
    const int lane = threadIdx.x & 63;
    *reinterpret_cast<uint4*>(a.out + br * kDV + 8 * lane) = make_uint4(0, 0, 0, 0);
    if (a.lse && lane == 0) {
      const int qi = row / a.h_q, h = row - qi * a.h_q;
      a.lse[((size_t)b * a.h_q + h) * a.s_q + qi] = kNegInf;
    }
    return;
  }
  // Shares holding tile p0 and tile p1 - 1: the largest w with start(w) <= t.
  const int w_lo = (int)(((p0 + 1) * (uint64_t)n - 1) / T);
  const int w_hi = (int)((p1 * (uint64_t)n - 1) / T);
  if (w_lo == w_hi) return;
  // Pieces: share w_lo's last slot (its first if the request starts the
  // share), then the first slot of each later share up to w_hi.
  const int first_slot = 2 * w_lo + (p0 > share_start(T, w_lo, n) ? 1 : 0);
  merge_row(a, br, w_hi - w_lo + 1, [&](int i) {
    return (size_t)(i == 0 ? first_slot : 2 * (w_lo + i)) * a.R + row;
  });
}

}  // namespace mla

extern "C" size_t mla_decode_workspace_bytes(int B, int s_q, int h_q, int num_splits) {
  if (B <= 0 || s_q <= 0 || h_q <= 0 || num_splits <= 1) return 0;
  return (size_t)B * s_q * h_q * num_splits * (mla::kDV + 2) * sizeof(float);
}

extern "C" int mla_decode_pick_num_splits(int B, int s_q, int h_q, int block_size, int max_blocks,
                                          int num_cus) {
  constexpr int64_t kMinChunk = 256;
  if (B < 1 || s_q < 1 || h_q < 1 || block_size < 1 || max_blocks < 1) return 0;
  if (num_cus <= 0 && (num_cus = gqa::device_cu_count()) <= 0) return 0;
  const int64_t groups =
      (int64_t)B * (((int64_t)s_q * h_q + mla::kRowsPerGroup - 1) / mla::kRowsPerGroup);
  int64_t ns = (num_cus + groups - 1) / groups;
  const int64_t s_max = (int64_t)max_blocks * block_size;
  ns = std::min<int64_t>(ns, std::max<int64_t>(1, s_max / kMinChunk));
  ns = std::min<int64_t>(ns, MLA_DECODE_MAX_SPLITS);
  return (int)std::max<int64_t>(ns, 1);
}

namespace {

// Checks the launch arguments and fills the kernel arguments; hipSuccess or
// hipErrorInvalidValue. A zero-request batch returns hipSuccess with a->B 0.
hipError_t make_args(mla::MlaArgs* a, const uint16_t* q, const uint16_t* kv_cache,
                     const int* block_table, const int* seq_lens, uint16_t* out, float* lse,
                     int B, int s_q, int h_q, int block_size, int max_blocks, float scale,
                     int causal, int num_splits, void* workspace, size_t workspace_bytes) {
  if (B < 0 || B > 65535 || s_q < 1 || h_q < 1 || block_size < 1 || max_blocks < 1)
    return hipErrorInvalidValue;
  const int64_t R = (int64_t)s_q * h_q;
  if (R > (int64_t(1) << 20) || (int64_t)B * R > (int64_t(1) << 31)) return hipErrorInvalidValue;
  if ((int64_t)block_size * max_blocks >= (int64_t(1) << 31)) return hipErrorInvalidValue;
  if (num_splits < 1 || num_splits > MLA_DECODE_MAX_SPLITS) return hipErrorInvalidValue;
  a->B = B;
  if (B == 0) return hipSuccess;
  if (!q || !kv_cache || !block_table || !seq_lens || !out) return hipErrorInvalidValue;
  a->q = q;
  a->kv = kv_cache;
  a->block_table = block_table;
  a->seq_lens = seq_lens;
  a->out = out;
  a->lse = lse;
  a->ws_acc = a->ws_m = a->ws_l = nullptr;
  a->pre = nullptr;
  a->first = nullptr;
  a->nshare = 0;
  a->s_q = s_q;
  a->h_q = h_q;
  a->R = (int)R;
  a->block_size = block_size;
  a->max_blocks = max_blocks;
  a->num_splits = num_splits;
  a->causal = causal ? 1 : 0;
  a->bs_div = gqa::make_fastdiv((uint32_t)block_size);
  a->scale_log2e = (float)((double)scale * 1.4426950408889634);
  if (num_splits > 1) {
    if (!workspace || ((uintptr_t)workspace & 15) != 0 ||
        workspace_bytes < mla_decode_workspace_bytes(B, s_q, h_q, num_splits))
      return hipErrorInvalidValue;
    const size_t states = (size_t)B * R * num_splits;
    a->ws_acc = static_cast<float*>(workspace);
    a->ws_m = a->ws_acc + states * mla::kDV;
    a->ws_l = a->ws_m + states;
  }
  return hipSuccess;
}

hipError_t launch_splitkv(const mla::MlaArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)((a.R + mla::kRowsPerGroup - 1) / mla::kRowsPerGroup), a.B,
                  a.num_splits);
  if (a.block_size % mla::kTile == 0)
    hipLaunchKernelGGL(mla::mla_decode_kernel<true>, grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(mla::mla_decode_kernel<false>, grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_combine(const mla::MlaArgs& a, hipStream_t stream) {
  const size_t rows = (size_t)a.B * a.R;
  hipLaunchKernelGGL(mla::mla_decode_merge_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                     stream, a);
  return hipGetLastError();
}

}  // namespace

extern "C" int mla_decode_launch(const uint16_t* q, const uint16_t* kv_cache, const int* block_table,
                                 const int* seq_lens, uint16_t* out, float* lse, int B, int s_q,
                                 int h_q, int block_size, int max_blocks, float scale, int causal,
                                 int num_splits, void* workspace, size_t workspace_bytes,
                                 hipStream_t stream) {
  mla::MlaArgs a;
  hipError_t err = make_args(&a, q, kv_cache, block_table, seq_lens, out, lse, B, s_q, h_q,
                             block_size, max_blocks, scale, causal, num_splits, workspace,
                             workspace_bytes);
  if (err != hipSuccess || a.B == 0) return err;
  err = launch_splitkv(a, stream);
  if (err != hipSuccess || num_splits == 1) return err;
  return launch_combine(a, stream);
}

extern "C" int mla_decode_splitkv_launch(const uint16_t* q, const uint16_t* kv_cache,
                                         const int* block_table, const int* seq_lens,
                                         uint16_t* out, float* lse, int B, int s_q, int h_q,
                                         int block_size, int max_blocks, float scale, int causal,
                                         int num_splits, void* workspace, size_t workspace_bytes,
                                         hipStream_t stream) {
  mla::MlaArgs a;
  hipError_t err = make_args(&a, q, kv_cache, block_table, seq_lens, out, lse, B, s_q, h_q,
                             block_size, max_blocks, scale, causal, num_splits, workspace,
                             workspace_bytes);
  if (err != hipSuccess || a.B == 0) return err;
  return launch_splitkv(a, stream);
}

extern "C" int mla_decode_combine_launch(void* workspace, size_t workspace_bytes, uint16_t* out,
                                         float* lse, int B, int s_q, int h_q, int num_splits,
                                         hipStream_t stream) {
  if (num_splits < 2) return hipErrorInvalidValue;
  // The combine kernel reads only the workspace and writes out and lse; the
  // other arguments only size the grid, so placeholders stand in for the
  // split kernel's inputs.
  static const uint16_t kNone = 0;
  static const int kNoInt = 0;
  mla::MlaArgs a;
  hipError_t err = make_args(&a, &kNone, &kNone, &kNoInt, &kNoInt, out, lse, B, s_q, h_q, 1, 1,
                             1.f, 0, num_splits, workspace, workspace_bytes);
  if (err != hipSuccess || a.B == 0) return err;
  return launch_combine(a, stream);
}

namespace {

constexpr int kMaxShares = 8192;

// Shares per row group of a balanced launch: num_workgroups (<= 0: the
// device's CU count) spread over the ceil(R / 128) row groups.
int balanced_shares(int s_q, int h_q, int num_workgroups) {
  if (num_workgroups <= 0 && (num_workgroups = gqa::device_cu_count()) <= 0) return 0;
  const int64_t rg = ((int64_t)s_q * h_q + mla::kRowsPerGroup - 1) / mla::kRowsPerGroup;
  return (int)std::min<int64_t>(kMaxShares, std::max<int64_t>(1, num_workgroups / rg));
}

size_t align16(size_t x) { return (x + 15) & ~size_t(15); }

}  // namespace

extern "C" size_t mla_decode_balanced_workspace_bytes(int B, int s_q, int h_q, int num_workgroups) {
  if (B <= 0 || s_q <= 0 || h_q <= 0) return 0;
  const int n = balanced_shares(s_q, h_q, num_workgroups);
  if (n <= 0) return 0;
  const size_t states = (size_t)2 * n * s_q * h_q;
  return align16(states * (mla::kDV + 2) * sizeof(float)) + align16((size_t)(B + 2) * 8) +
         (size_t)n * sizeof(int);
}

extern "C" int mla_decode_balanced_launch(const uint16_t* q, const uint16_t* kv_cache,
                                          const int* block_table, const int* seq_lens,
                                          uint16_t* out, float* lse, int B, int s_q, int h_q,
                                          int block_size, int max_blocks, float scale, int causal,
                                          int num_workgroups, void* workspace,
                                          size_t workspace_bytes, hipStream_t stream) {
  mla::MlaArgs a;
  hipError_t err = make_args(&a, q, kv_cache, block_table, seq_lens, out, lse, B, s_q, h_q,
                             block_size, max_blocks, scale, causal, 1, nullptr, 0);
  if (err != hipSuccess || a.B == 0) return err;
  const int n = balanced_shares(s_q, h_q, num_workgroups);
  const size_t need = mla_decode_balanced_workspace_bytes(B, s_q, h_q, num_workgroups);
  if (n <= 0 || !workspace || ((uintptr_t)workspace & 15) != 0 || workspace_bytes < need)
    return hipErrorInvalidValue;
  const size_t states = (size_t)2 * n * a.R;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  a.ws_acc = reinterpret_cast<float*>(ws);
  a.ws_m = a.ws_acc + states * mla::kDV;
  a.ws_l = a.ws_m + states;
  uint64_t* pre = reinterpret_cast<uint64_t*>(ws + align16(states * (mla::kDV + 2) * sizeof(float)));
  int* first = reinterpret_cast<int*>(reinterpret_cast<uint8_t*>(pre) + align16((size_t)(B + 2) * 8));
  a.pre = pre;
  a.first = first;
  a.nshare = n;
  hipLaunchKernelGGL(mla::mla_plan_kernel, dim3(1), dim3(256), 0, stream, a, pre, first);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  const unsigned rg = (unsigned)((a.R + mla::kRowsPerGroup - 1) / mla::kRowsPerGroup);
  if (block_size % mla::kTile == 0)
    hipLaunchKernelGGL(mla::mla_decode_balanced_kernel<true>, dim3(n, rg), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(mla::mla_decode_balanced_kernel<false>, dim3(n, rg), dim3(256), 0, stream, a);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  const size_t rows = (size_t)B * a.R;
  hipLaunchKernelGGL(mla::mla_decode_balanced_merge_kernel, dim3((unsigned)((rows + 3) / 4)),
                     dim3(256), 0, stream, a);
  return hipGetLastError();
}

