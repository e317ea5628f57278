// MLA absorbed-path paged decode for gfx950 (the reference's roadmap item K2,
// README.md:405-408): every query row (s_q x h_q of a request) attends over
// one shared latent cache of 576-dim rows; values are the rows' first 512
// dims. Semantics and layouts: include/mla_decode.h.
//
// Work decomposition. A workgroup of 8 waves (two per SIMD) owns 128 query
// rows (a row group) of one request and a range of its tokens. All rows share
// the cache rows, so each 32-token tile (36 KiB) is read from HBM once per
// workgroup: the four PV-first waves copy it, HBM -> LDS
// (global_load_lds_dwordx4, no registers), into a ring of kDepth slots, and
// every wave computes from LDS. Two launches share this tile walk (mla_piece):
//   fixed splits  grid (row groups, B, num_splits), split s of each request;
//   balanced      one workgroup per CU and row group, each taking an equal
//                 share of the batch's request-ordered tiles (each
//                 workgroup plans its share from seq_lens on the device),
//                 walked piece by piece; requests cut between shares are
//                 merged after.
//
// The two matrix products of a tile are split between the waves along
// different axes, which keeps each wave's registers at what two waves per
// SIMD can hold (256):
//   QK^T + softmax  wave w scores its 16 query rows 16w .. 16w + 15 against
//          the tile's 32 tokens (Q^T of those rows in registers) and writes
//          the rows' bf16 probabilities to a P buffer in LDS;
//   PV     wave w accumulates O[all 128 rows][dims 64w .. 64w + 63] from the
//          P buffer and the tile's column block w (128 fp32 accumulators).
// A tile's PV needs every wave's probabilities, so the walk is pipelined over
// intervals: interval s scores tile s into P buffer s % 2 while accumulating
// tile s - 1 from P buffer (s - 1) % 2, with one workgroup barrier per
// interval. Waves 0-3 accumulate first and score second, waves 4-7 the other
// way round, so the two waves of a SIMD keep the matrix unit busy through each
// other's softmax. The ring holds tile s - 1 (PV), tile s (QK), tile s + 1
// (landing) and tile s + 2 (copied during interval s): 4 x 36 KiB + 2 x 8 KiB
// of P = 160 KiB, the whole LDS.
//
// LDS tile layout: 4 row blocks of 8 tokens, each 9 column blocks of 1 KiB
// (8 rows x 128 bytes = 64 dims), so column block cb of row block rb8 is the
// tile's 1 KiB block 9 rb8 + cb; within a column block, row r sits at 128 r and
// its 16-byte chunk c at position c ^ chunk_swz(rb8, r). Each copy
// instruction fills one column block: 8 lanes per row read that row's 128
// contiguous bytes from HBM (a copy of 16 rows x 64 bytes per instruction
// streamed at ~4.5 TB/s, 8 x 128 bytes at ~6.2 TB/s, measured on MI355X), and
// the swizzle only permutes lanes within a row. The swizzle makes both operand
// reads free of bank conflicts under the LDS rules measured on MI355X (64
// banks of 4 bytes; bank-conflict counters over single-pattern probes):
// ds_read_b128 serves a wave in 4 phases of 16 lanes, lane l in phase
// 2 (l / 32) + parity((l / 4) % 8) (lane 0 shares its phase with lanes 1-3,
// 12-15 and 20-27), free of conflicts when the phase's 16-byte bank quads
// (addr / 16) % 16 differ; ds_read_b64 and ds_read_b64_tr_b16 serve lanes
// 0-31 and 32-63, free when (addr / 8) % 32 differ.
//
//   QK^T   S^T[16 tok x 16 rows] = K[tok x 576] . Q^T[576 x 16 rows]: 18
//          v_mfma_f32_16x16x32_bf16 per 16-token group; A from LDS (lane:
//          token j, dims 32 kk + 8 g), B = Q^T in registers (lane: row j,
//          dims 32 kk + 8 g).
//   softmax on the C layout (lane: row j, tokens 16 tg + 4 g + e), base 2,
//          fp32, against a per-row reference max fixed at the row's first live
//          tile (see kRefSlack); P rounded to bf16, l sums the rounded values.
//          P buffer: row R at 64 R, 16-byte chunk c (tokens 8c .. 8c + 7) at
//          position c ^ (-(R / 4) % 4) (conflict-free ds_read_b128 A reads).
//   PV     O[16 rows x 16 dims] += P[16 rows x 32 tok] . V[32 tok x 16 dims]:
//          8 row blocks x 4 column blocks of v_mfma_f32_16x16x32_bf16, k-slot
//          8 g + e = token 8 g + e; A = one ds_read_b128 of the P buffer
//          (lane: row j, chunk g), B = two ds_read_b64_tr_b16 of the tile
//          (lane x of 16-lane group g supplies token 8 g + 4 h + x / 4, dims
//          16 nb + 4 (x % 4) .. +4; the transpose hands lane x the four tokens
//          of dim 16 nb + x).
//
// Splits and shares cut requests at multiples of 32 tokens; the merges fold
// the pieces in order (log-sum-exp), so results are bitwise reproducible.
#include "gqa_device.hpp"
#include "gqa_launch.hpp"
#include "mla_decode.h"

#include <algorithm>
#include <type_traits>

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
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kRowsPerWave = 16;                      // QK^T rows of a wave
constexpr int kRowsPerGroup = kWaves * kRowsPerWave;  // 128
constexpr int kRowBlocks = kRowsPerGroup / 16;        // 8 PV row blocks
constexpr int kTileBlocks = 2 * kKSteps;              // 36 blocks of 1 KiB
constexpr int kColBlocks = kD / 64;                   // 9 per row block of 8 tokens
constexpr int kRowBlockBytes = kColBlocks * 1024;
constexpr int kTileBytes = 4 * kRowBlockBytes;        // 36 KiB
// Copy instructions per wave per tile: blocks w, w + 8, ...; waves below
// kWavesHi take one more.
constexpr int kLoadsHi = (kTileBlocks + kWaves - 1) / kWaves;  // 5
constexpr int kLoadsLo = kTileBlocks / kWaves;                 // 4
constexpr int kWavesHi = kTileBlocks % kWaves;                 // 4
constexpr int kDepth = 4;                                      // ring slots
constexpr int kPBytes = kRowsPerGroup * kTile * 2;             // one P buffer, 8 KiB
constexpr int kLdsBytes = kDepth * kTileBytes + 2 * kPBytes;   // 160 KiB
constexpr int kNBw = kDV / kWaves / 16;                        // 4 PV column blocks per wave
static_assert(kDV / kWaves == 64, "wave w accumulates the tile's column block w");
static_assert(kTileBlocks == 4 * kColBlocks, "a tile is 4 row blocks of 9 column blocks");
static_assert(kLdsBytes <= 160 * 1024, "the ring and the P buffers fill the LDS");
static_assert(kWavesHi * 2 <= kWaves, "the waves that take kLoadsHi copies accumulate first");
#ifndef MLA_COPY_WAVES
#define MLA_COPY_WAVES 4
#endif
// Waves that issue a tile's copies: only the 4 PV-first waves (9 copies
// each; a copy instruction's issue stalls its wave while the address unit
// works through the others), which leaves the QK-first waves free to start
// their QK^T right after the barrier; or (MLA_COPY_WAVES=8) all 8 waves.
constexpr int kCopyWaves = MLA_COPY_WAVES;
static_assert(kCopyWaves == 8 || kCopyWaves == 4, "copy waves");
constexpr int kCopyStride = kCopyWaves / 2;  // copy waves per row-block parity
constexpr int kCopyHi = kCopyWaves == 8 ? kLoadsHi : kTileBlocks / 4;  // copies of waves < 4
constexpr int kCopyLo = kCopyWaves == 8 ? kLoadsLo : 0;                // copies of waves >= 4

// Position XOR of row r's 16-byte chunks in a column block of row block rb8
// (the table depends on rb8's parity; found by a search over tables that
// checks both operand reads against the measured LDS phase rules above).
__device__ __forceinline__ int chunk_swz(int rb8, int r) {
  return (int)((0x0052246637751143ull >> (4 * (8 * (rb8 & 1) + r))) & 7u);
}

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
  uint64_t* pre;        // balanced launch: tile prefix sums [B + 2] (written by the split kernel)
  int B, s_q, h_q, R, block_size, max_blocks, num_splits, causal, nshare;
  FastDiv bs_div;
  float scale_log2e;
};

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4& u) {
  return __builtin_bit_cast(bf16x8_t, u);
}

// A row's probabilities are taken relative to a reference max that is set by
// the first tile holding a live key of the row and then kept: rescaling the
// 128 x 64 fp32 accumulators of a wave (half of its registers) on every new
// max would cost more than the tile's matrix work, and any conditional update
// of them inside the tile loop makes the compiler copy them on every tile.
// Probabilities stay below 2^kRefSlack; if a later tile beats a row's
// reference by more, the workgroup runs its split a second time against the
// rows' true maxima (the values are exact either way; only that split's time
// doubles).
constexpr float kRefSlack = 32.f;
// LDS operand reads run ahead of their use: QK reads through a ring of
// kKRing single-read slots (each read kKRing - 1 MFMAs ahead), PV P-operand
// reads kPAhead row blocks (4 MFMAs each) ahead.
constexpr int kKRing = 5;

// Profiling build (build.py --variant NAME --define MLA_PHASE_TIMING=1; read
// by bench/mla_phases.py): every wave stamps the shader clock (s_memtime) at
// the phase boundaries of its tile intervals and pieces and adds the cycles
// to its row of mla_phase_cycles (one row per wave of the first 256
// workgroups; columns kPh*). The stamps wait for the scalar cache, which
// costs a few percent; the shipped library is built without them.
#ifndef MLA_PHASE_TIMING
#define MLA_PHASE_TIMING 0
#endif
enum PhaseCol {
  kPhCopies, kPhFirst, kPhQK, kPhSoftmax, kPhSecond, kPhBarrier, kPhIntervals,  // full intervals
  kPhQLoad, kPhPrologue, kPhKind0, kPhKind2, kPhVote, kPhEpilogue, kPhPieces,    // pieces
  kPhKernel, kPhKernelRealtime, kPhCols
};
#if MLA_PHASE_TIMING
__device__ unsigned long long mla_phase_cycles[2048][kPhCols];
#define MLA_STAMP(x)                                                    \
  __builtin_amdgcn_sched_barrier(0);                                    \
  const uint32_t x = (uint32_t)__builtin_amdgcn_s_memtime();           \
  __builtin_amdgcn_sched_barrier(0)
#define MLA_PHASE_ADD(col, from, to) (ph[col] += (to) - (from))
#else
#define MLA_STAMP(x)
#define MLA_PHASE_ADD(col, from, to)
#endif
constexpr int kPAhead = 2;

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
// (they complete in issue order) and its LDS writes are done, then joins the
// workgroup barrier; LDS reads and writes are not moved across it.
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

// After a pass, P buffer 1 (first written in the second interval of a pass,
// two barriers after any pass starts) holds the restart votes and the rows'
// final sums.
constexpr int kStatL = 0;    // 128 floats: row sums
constexpr int kVotes = 512;  // 8 ints

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) u32x4_t lds_u32x4_t;
typedef __attribute__((address_space(3))) u32x2_t lds_u32x2_t;

// LDS accesses by 32-bit LDS byte address.
__device__ __forceinline__ u32x4_t lds_load16(uint32_t addr) {
  return *(const lds_u32x4_t*)(uintptr_t)addr;
}
__device__ __forceinline__ void lds_store8(uint32_t addr, u32x2_t v) {
  *(lds_u32x2_t*)(uintptr_t)addr = v;
}
__device__ __forceinline__ bf16x4_t lds_load_tr(uint32_t addr) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)(uintptr_t)addr);
}
__device__ __forceinline__ bf16x8_t as_bf16x8(const u32x4_t& u) {
  return __builtin_bit_cast(bf16x8_t, u);
}

// Hands x back through an empty asm statement, so that the compiler treats it
// as a new value: applied to the lane's operand offsets at the top of every
// interval, it keeps values derived from them (offset ^ constant, one per
// matrix step) from being hoisted out of the tile loop, where they would
// outgrow the register budget of two waves per SIMD.
__device__ __forceinline__ void refresh(uint32_t& x) { asm volatile("" : "+v"(x)); }

// The workgroup's 128 query rows (row group rg) of request b against tokens
// [seg_start, seg_end) of the request's S live tokens. Every wave of the
// workgroup calls it with the same arguments (its barriers are workgroup-wide).
template <bool kBlockUniform>
__device__ __forceinline__ void mla_piece(const MlaArgs& a, uint8_t* smem, int b, int rg, int S,
                                          int seg_start, int seg_end, PieceOut po) {
  typedef __attribute__((address_space(3))) uint8_t lds_u8;
  // Every lane-dependent value below derives from tid, refreshed here so that
  // none of them is hoisted out of a caller's loop over pieces.
  MLA_STAMP(ph_start);
#if MLA_PHASE_TIMING
  uint32_t ph[kPhCols] = {};
  uint32_t ph_mid = 0, ph_pro = 0;
#endif
  uint32_t tid = threadIdx.x;
  refresh(tid);
  const int lane = (int)(tid & 63);
  const int w = __builtin_amdgcn_readfirstlane((int)(tid >> 6));
  const int j = lane & 15, g = lane >> 4;
  const uint32_t smem_lds = (uint32_t)(uintptr_t)(lds_u8*)smem;
  const uint32_t pbuf_lds = smem_lds + kDepth * kTileBytes;  // P buffer t at + t * kPBytes
  uint8_t* const pbuf1 = smem + kDepth * kTileBytes + kPBytes;

  // Copies. Wave w copies row blocks of parity par = w % 2 only (row blocks
  // par and par + 2: 18 column blocks m, rb8 = par + 2 (m / 9), cb = m % 9),
  // taking m = w / 2 + 2 i (i < 9, m < 18): 9 copies for each of waves 0-3,
  // none for waves 4-7 (with MLA_COPY_WAVES=8: m = w / 2 + 4 i, 5 copies for
  // waves 0-3, 4 for waves 4-7). Lane x fills row cr = x / 8 of a column block, position x % 8,
  // from that row's chunk (x % 8) ^ chunk_swz(par, cr): one source offset
  // per lane, ro (the row's offset; ro & 0x70 is its chunk's offset in row 0).
  const int par = w & 1, cu = w >> 1;
  uint32_t ro = (uint32_t)((lane >> 3) * kD + 8 * ((lane & 7) ^ chunk_swz(par, lane >> 3))) * 2u;
  // Tile-relative LDS offsets of this lane's operands (plus per-step
  // immediates or XORs; a slot's address has its low 10 bits clear, so a XOR
  // applies to slot + offset as well):
  //  QK A operand of token 16 tg + j, chunk 4 par + g of column block kk / 2
  //    (k-step parity flips bit 6: ^ 64; token group 1 is two row blocks on);
  //  PV B operand of row block g, column block w, rows 4 h + j / 4, chunk
  //    2 nb + (j % 4) / 2, half j % 2 (nb flips bits 5-6: ^ 32 nb);
  //  P buffer: A operand row 16 rb + j, chunk g (+ 1 KiB per row block); the
  //    lane's probabilities, row 16 w + j, chunks 2 tg + g / 2, half g % 2
  //    (tg flips bit 5: ^ 32).
  uint32_t qoff = (uint32_t)((j >> 3) * kRowBlockBytes + (j & 7) * 128 +
                             16 * (g ^ chunk_swz(j >> 3, j & 7)));
  uint32_t vx0, vx1;
  {
    const int r0 = j >> 2, r1 = 4 + (j >> 2);
    const int base = g * kRowBlockBytes + w * 1024 + 8 * (j & 1);
    vx0 = (uint32_t)(base + r0 * 128 + 16 * (((j & 3) >> 1) ^ chunk_swz(g, r0)));
    vx1 = (uint32_t)(base + r1 * 128 + 16 * (((j & 3) >> 1) ^ chunk_swz(g, r1)));
  }
  // (The copy row and the P buffer offsets are recomputed from tid where
  // they are used: three fewer registers held through the tile loop.)
  auto lane_cr = [&]() -> int { return (int)((tid >> 3) & 7); };
  auto pr_off = [&]() -> uint32_t {
    const uint32_t jj = tid & 15, gg = (tid >> 4) & 3;
    return jj * 64 + 16 * (gg ^ (-(jj >> 2) & 3));
  };
  auto pw_off = [&]() -> uint32_t {
    const uint32_t jj = tid & 15, gg = (tid >> 4) & 3;
    return (uint32_t)w * 1024 + jj * 64 + 16 * ((gg >> 1) ^ (-(jj >> 2) & 3)) + 8 * (gg & 1);
  };

  // Waves whose rows all lie past R score zero queries (their results are not
  // stored): a wave-dependent branch around the tile work would make the
  // compiler copy the accumulators on every tile.
  const int row0 = rg * kRowsPerGroup + w * kRowsPerWave;
  const int ntiles = (seg_end - seg_start + kTile - 1) / kTile;

  // Q^T as the B operand, all 18 k-steps in registers (lane: row j, dims
  // 32 kk + 8 g); and the lane's key limit for its row j, less 4 g (token
  // 16 tg + 4 g + e of the tile at ts is live iff 16 tg + e < lim4 - ts).
  uint4 qf[kKSteps];
  int lim4;
  {
    const int r = row0 + j;
    const bool live = r < a.R;
    const uint16_t* qrow = a.q + ((size_t)b * a.R + (live ? r : 0)) * kD + 8 * g;
#pragma unroll
    for (int kk = 0; kk < kKSteps; ++kk)
      qf[kk] = live ? *reinterpret_cast<const uint4*>(qrow + 32 * kk) : make_uint4(0, 0, 0, 0);
    const int qi = live ? r / a.h_q : 0;
    lim4 = min(seg_end, a.causal ? S - (a.s_q - 1 - qi) : S) - 4 * g;
  }
  // Let the Q loads land here: a wait left to their first use would sit inside
  // the tile loop, where it would also wait for every tile copy in flight.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)

  MLA_STAMP(ph_q);
  MLA_PHASE_ADD(kPhQLoad, ph_start, ph_q);
  const int* bt = a.block_table + (size_t)b * a.max_blocks;
  // The table is read-only for the launch; through the constant address space
  // the uniform block-id loads become scalar loads.
  const __attribute__((address_space(4))) int* btc =
      (const __attribute__((address_space(4))) int*)bt;
  const int bs = a.block_size;

  // Staging of tile k into ring slot k % kDepth. Tokens at or past seg_end
  // read the tile's first token instead (masked later), so nothing outside
  // the request's live cache rows is touched. Block ids come from scalar
  // loads, which keeps the vector memory counter for the copies alone. A
  // refill goes out at the start of an interval, right after the barrier
  // that freed its slot; its block id is loaded one interval ahead, before
  // that barrier, so that the scalar-load latency overlaps the wait for the
  // landing tile.
  auto block_id = [&](int k) -> int {
    return btc[gqa::fastdiv((uint32_t)(seg_start + kTile * k), a.bs_div)];
  };
  auto stage = [&](int k, int id) {
    const int ts = seg_start + kTile * k;
    const uint32_t slot = smem_lds + (uint32_t)(k % kDepth) * kTileBytes;
    if constexpr (kBlockUniform) {
      // 32 tokens from a 32-aligned start share one block: a uniform base row.
      const uint32_t lb = gqa::fastdiv((uint32_t)ts, a.bs_div);
      const uint16_t* base = a.kv + ((size_t)id * bs + (ts - (int)lb * bs)) * kD;
      const int nvalid = seg_end - ts;
      auto copy = [&](int i) {
        const int m = cu + kCopyStride * i, hi = m >= kColBlocks ? 1 : 0;
        const int rb8 = par + 2 * hi, cb = m - kColBlocks * hi;
        // (The row block's offset stays in the lane offset: a row past
        // seg_end must land on the tile's first row, not the block's.)
        const uint32_t voff = lane_cr() < nvalid - 8 * rb8 ? ro + (uint32_t)(8 * rb8 * kD * 2)
                                                            : (ro & 0x70u);
        load_to_lds(base + 64 * cb, voff,
                    __builtin_amdgcn_readfirstlane(slot + (kColBlocks * rb8 + cb) * 1024));
      };
      if constexpr (kCopyWaves == 8) {
#pragma unroll
        for (int i = 0; i < kLoadsLo; ++i) copy(i);
        if (w < kWavesHi) copy(kLoadsLo);
      } else if (w < kWavesHi) {
#pragma unroll
        for (int i = 0; i < kCopyHi; ++i) copy(i);
      }
    } else {
      // The tile's tokens span blocks lb_lo .. lb_hi: fetch their ids with
      // uniform loads and let each lane take its own rows (one per row block
      // of the wave's parity).
      const int t_hi = min(ts + kTile, seg_end) - 1;
      const int lb_lo = (int)gqa::fastdiv((uint32_t)ts, a.bs_div);
      const int lb_hi = (int)gqa::fastdiv((uint32_t)t_hi, a.bs_div);
      int tok[2], lbl[2];
      size_t row[2] = {0, 0};
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        const int t = 8 * (par + 2 * x) + lane_cr();
        tok[x] = ts + t < seg_end ? t : 0;
        lbl[x] = (int)gqa::fastdiv((uint32_t)(ts + tok[x]), a.bs_div);
      }
      for (int q = lb_lo; q <= lb_hi; ++q) {
        const size_t bid = (size_t)btc[q];
#pragma unroll
        for (int x = 0; x < 2; ++x) row[x] = lbl[x] == q ? bid : row[x];
      }
      const uint16_t* src[2];
#pragma unroll
      for (int x = 0; x < 2; ++x)
        src[x] = a.kv + (row[x] * bs + (ts + tok[x] - lbl[x] * bs)) * kD + ((ro & 0x70u) >> 1);
      auto copy = [&](int i) {
        const int m = cu + kCopyStride * i, hi = m >= kColBlocks ? 1 : 0;
        const int rb8 = par + 2 * hi, cb = m - kColBlocks * hi;
        load_to_lds((hi ? src[1] : src[0]) + 64 * cb,
                    __builtin_amdgcn_readfirstlane(slot + (kColBlocks * rb8 + cb) * 1024));
      };
      if constexpr (kCopyWaves == 8) {
#pragma unroll
        for (int i = 0; i < kLoadsLo; ++i) copy(i);
        if (w < kWavesHi) copy(kLoadsLo);
      } else if (w < kWavesHi) {
#pragma unroll
        for (int i = 0; i < kCopyHi; ++i) copy(i);
      }
    }
  };
  // End of an interval: the next tile must have landed (with a refill in
  // flight, this wave's copies of it stay outstanding), then the barrier.
  auto publish = [&](bool refill) {
    if (!refill)
      publish_barrier<0>();
    else if (w < kWavesHi)
      publish_barrier<kCopyHi>();
    else
      publish_barrier<kCopyLo>();
  };

  f32x4_t o[kRowBlocks][kNBw];
  float lsum = 0.f;
  float mref = kNegInf;   // row j's reference max (log2 units)
  float mtrue = kNegInf;  // row j's max over the split so far (lane-local)
  bool beaten = false;    // some row's max beat its reference

  // QK^T and softmax of tile s into P buffer s % 2.
  auto score = [&](int s) {
    const uint32_t T = smem_lds + (uint32_t)(s % kDepth) * kTileBytes;
    const int ts = seg_start + kTile * s;
    // c[tg][e] = score of token 16 tg + 4 g + e for row j. The tile's 36
    // operand reads (read n: k-step n / 2, token group n % 2) cycle through a
    // ring of kKRing registers, each issued kKRing - 1 MFMAs ahead of its use
    // (the scheduling barriers keep the compiler from sinking them).
    const uint32_t qa = T + qoff;
    auto read_k = [&](int n) -> u32x4_t {
      const int kk = n >> 1, tg = n & 1;
      return lds_load16((qa ^ (64u * (kk & 1))) + 2 * kRowBlockBytes * tg + 1024 * (kk >> 1));
    };
    f32x4_t c[2];
#pragma unroll
    for (int tg = 0; tg < 2; ++tg) c[tg] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    u32x4_t kr[kKRing];
#pragma unroll
    for (int n = 0; n < kKRing - 1; ++n) kr[n] = read_k(n);
#pragma unroll
    for (int n = 0; n < 2 * kKSteps; ++n) {
      // The slot refilled here was read by the previous MFMA.
      if (n + kKRing - 1 < 2 * kKSteps) kr[(n + kKRing - 1) % kKRing] = read_k(n + kKRing - 1);
      __builtin_amdgcn_sched_barrier(0);
      c[n & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kr[n % kKRing]),
                                                         as_bf16x8(qf[n >> 1]), c[n & 1], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    // Probabilities against the reference max, rounded to bf16 (l sums the
    // rounded values). The lane's tokens are live iff 16 tg + e < d; a tile
    // where that holds for every lane (d >= 20 everywhere) skips the masking.
    const int d = lim4 - ts;
#if MLA_PHASE_TIMING
    {
      MLA_STAMP(ph_m);
      ph_mid = ph_m;
    }
#endif
    const bool partial = __builtin_amdgcn_ballot_w64(d < 20) != 0;
    float sc[2][4];
    float mx = kNegInf;
    if (partial) {
#pragma unroll
      for (int tg = 0; tg < 2; ++tg)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sc[tg][e] = 16 * tg + e < d ? c[tg][e] * a.scale_log2e : kNegInf;
          mx = fmaxf(mx, sc[tg][e]);
        }
    } else {
#pragma unroll
      for (int tg = 0; tg < 2; ++tg)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sc[tg][e] = c[tg][e] * a.scale_log2e;
          mx = fmaxf(mx, sc[tg][e]);
        }
    }
    // mx is this lane's max (its 8 tokens of row j). The row's first live tile
    // sets the reference (nothing is accumulated before it, so nothing needs
    // rescaling); the row's four lanes agree on it.
    mref = mref == kNegInf ? row_max(mx) : mref;
    beaten |= mx > mref + kRefSlack;
    mtrue = fmaxf(mtrue, mx);
    const float base = mref == kNegInf ? 0.f : mref;
    const uint32_t pw = pbuf_lds + (uint32_t)(s & 1) * kPBytes + pw_off();
    float psum = 0.f;
#pragma unroll
    for (int tg = 0; tg < 2; ++tg) {
      uint32_t wd[2];
#pragma unroll
      for (int e = 0; e < 4; e += 2) {
        const gqa::bf16x2_t pb = __builtin_convertvector(
            (float __attribute__((ext_vector_type(2)))){exp2_fast(sc[tg][e] - base),
                                                        exp2_fast(sc[tg][e + 1] - base)},
            gqa::bf16x2_t);
        wd[e / 2] = __builtin_bit_cast(uint32_t, pb);
        psum = gqa::dot2_bf16(wd[e / 2], 0x3F803F80u, psum);  // + both values (x 1.0)
      }
      lds_store8(pw ^ (32u * tg), u32x2_t{wd[0], wd[1]});
    }
    lsum += psum;
  };

  // PV of tile s from P buffer s % 2: o[rb][nb] += P[rows 16 rb .. +16][32
  // tok] . V[32 tok][dims 64 w + 16 nb .. +16].
  auto accumulate = [&](int s) {
    const uint32_t T = smem_lds + (uint32_t)(s % kDepth) * kTileBytes;
    const uint32_t va0 = T + vx0, va1 = T + vx1;
    const uint32_t pa_addr = pbuf_lds + (uint32_t)(s & 1) * kPBytes + pr_off();
    bf16x8_t vv[kNBw];
#pragma unroll
    for (int nb = 0; nb < kNBw; ++nb) {
      const bf16x4_t v0 = lds_load_tr(va0 ^ (32u * nb));
      const bf16x4_t v1 = lds_load_tr(va1 ^ (32u * nb));
      vv[nb] = bf16x8_t{v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
    }
    u32x4_t pa[kPAhead + 1];
#pragma unroll
    for (int rb = 0; rb < kPAhead; ++rb) pa[rb] = lds_load16(pa_addr + 1024 * rb);
#pragma unroll
    for (int rb = 0; rb < kRowBlocks; ++rb) {
      if (rb + kPAhead < kRowBlocks)
        pa[(rb + kPAhead) % (kPAhead + 1)] = lds_load16(pa_addr + 1024 * (rb + kPAhead));
      __builtin_amdgcn_sched_barrier(0);
      const bf16x8_t pv = as_bf16x8(pa[rb % (kPAhead + 1)]);
#pragma unroll
      for (int nb = 0; nb < kNBw; ++nb)
        o[rb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pv, vv[nb], o[rb][nb], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // One pass over the split's tiles, accumulating o and lsum against mref.
  // Interval kinds: 0 scores tile 0 only, 1 scores tile s and accumulates
  // tile s - 1, 2 accumulates the last tile only.
  auto pass = [&](auto pv_first) {
    constexpr bool kPVFirst = decltype(pv_first)::value;
    lsum = 0.f;
#pragma unroll
    for (int rb = 0; rb < kRowBlocks; ++rb)
#pragma unroll
      for (int nb = 0; nb < kNBw; ++nb) o[rb][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    if (ntiles == 0) return;
    int id_next = 0;
    auto interval = [&](auto kind, int s) {
      constexpr int kKind = decltype(kind)::value;
      constexpr bool kQK = kKind != 2, kPV = kKind != 0;
      refresh(tid);
      refresh(ro);
      refresh(qoff);
      refresh(vx0);
      refresh(vx1);
      MLA_STAMP(ph0);
      const bool refill = kQK && s + 2 < ntiles;
      if (refill) stage(s + 2, id_next);
      __builtin_amdgcn_sched_barrier(0);
      MLA_STAMP(ph1);
      if constexpr (kPV && kPVFirst) accumulate(s - 1);
      MLA_STAMP(ph2);
      if constexpr (kQK) {
        // The QK-first wave of each SIMD scores at raised issue priority: its
        // softmax (VALU) then overlaps the other wave's matrix work, instead
        // of both waves' QK^T contending for the LDS and both softmaxes
        // leaving the matrix unit idle.
        if constexpr (!kPVFirst) __builtin_amdgcn_s_setprio(2);
        score(s);
        if constexpr (!kPVFirst) __builtin_amdgcn_s_setprio(0);
      }
      MLA_STAMP(ph3);
      if constexpr (kPV && !kPVFirst) accumulate(s - 1);
      // The block id of the next interval's refill, loaded here so that its
      // latency overlaps the wait below.
      if constexpr (kBlockUniform) {
        if (s + 3 < ntiles) id_next = block_id(s + 3);
      }
      MLA_STAMP(ph4);
      publish(refill);
      MLA_STAMP(ph5);
#if MLA_PHASE_TIMING
      if constexpr (kKind == 1) {
        MLA_PHASE_ADD(kPhCopies, ph0, ph1);
        MLA_PHASE_ADD(kPhFirst, ph1, ph2);
        MLA_PHASE_ADD(kPhQK, ph2, ph_mid);
        MLA_PHASE_ADD(kPhSoftmax, ph_mid, ph3);
        MLA_PHASE_ADD(kPhSecond, ph3, ph4);
        MLA_PHASE_ADD(kPhBarrier, ph4, ph5);
        ph[kPhIntervals] += 1;
      } else if constexpr (kKind == 0) {
        MLA_PHASE_ADD(kPhKind0, ph0, ph5);
      } else {
        MLA_PHASE_ADD(kPhKind2, ph0, ph5);
      }
#endif
    };
    // Prologue: tiles 0 and 1 in flight; tile 0 published.
    stage(0, kBlockUniform ? block_id(0) : 0);
    if (ntiles > 1) stage(1, kBlockUniform ? block_id(1) : 0);
    if constexpr (kBlockUniform) {
      if (ntiles > 2) id_next = block_id(2);
    }
    publish(ntiles > 1);
#if MLA_PHASE_TIMING
    {
      MLA_STAMP(ph_p);
      ph_pro = ph_p;
    }
#endif
    interval(std::integral_constant<int, 0>{}, 0);
    for (int s = 1; s < ntiles; ++s) interval(std::integral_constant<int, 1>{}, s);
    interval(std::integral_constant<int, 2>{}, ntiles);
  };
  auto run_pass = [&]() {
    if (w < kWaves / 2)
      pass(std::true_type{});
    else
      pass(std::false_type{});
  };

  run_pass();
  MLA_STAMP(ph_run);
  MLA_PHASE_ADD(kPhPrologue, ph_q, ph_pro);
  // A row whose max beat its reference by more than kRefSlack has overflowed
  // or lost precision: the workgroup (which stages tiles together) runs the
  // split again with every row's reference at its true max (probabilities
  // <= 1, so a second pass always suffices). The ballot is taken with the
  // whole wave active (each lane holds its own row's and tokens' flag); only
  // the store is lane 0's.
  int* const votes = reinterpret_cast<int*>(pbuf1 + kVotes);
  const bool wave_beaten = __builtin_amdgcn_ballot_w64(beaten) != 0;
  if (lane == 0) votes[w] = wave_beaten;
  __syncthreads();
  const uint4 va = *reinterpret_cast<const uint4*>(votes);
  const uint4 vb = *reinterpret_cast<const uint4*>(votes + 4);
  if ((va.x | va.y | va.z | va.w | vb.x | vb.y | vb.z | vb.w) != 0) {
    mref = row_max(mtrue);
    run_pass();
  }

  MLA_STAMP(ph_vote);
  MLA_PHASE_ADD(kPhVote, ph_run, ph_vote);
  // Row j's final l (lane (j, g) holds l over its own tokens), published to
  // every wave through the LDS; its owner writes the row's (m, l) or lse.
  float L = lsum + __shfl_xor(lsum, 16, 64);
  L += __shfl_xor(L, 32, 64);
  float* const stat_l = reinterpret_cast<float*>(pbuf1 + kStatL);
  if (g == 0) {
    stat_l[kRowsPerWave * w + j] = L;
    const int row = row0 + j;
    if (row < a.R) {
      if (po.direct) {
        if (a.lse) {
          const int qi = row / a.h_q, h = row - qi * a.h_q;
          a.lse[((size_t)b * a.h_q + h) * a.s_q + qi] = L > 0.f ? mref * kLn2 + logf(L) : kNegInf;
        }
      } else {
        const size_t sx = po.st_base + (size_t)row * po.st_stride;
        a.ws_m[sx] = L > 0.f ? mref * kLn2 : kNegInf;  // natural-log units
        a.ws_l[sx] = L;
      }
    }
  }
  __syncthreads();
  // This wave's o entries: rows 16 rb + 4 g + e, dims 64 w + 16 nb + j.
#pragma unroll
  for (int rb = 0; rb < kRowBlocks; ++rb) {
    const float4 L4 = *reinterpret_cast<const float4*>(stat_l + 16 * rb + 4 * g);
    const float Le[4] = {L4.x, L4.y, L4.z, L4.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = rg * kRowsPerGroup + 16 * rb + 4 * g + e;
      if (row >= a.R) continue;
      const size_t br = (size_t)b * a.R + row;
      if (po.direct) {
        const float inv = Le[e] > 0.f ? 1.f / Le[e] : 0.f;
        uint16_t* dst = a.out + br * kDV + 64 * w + j;
#pragma unroll
        for (int nb = 0; nb < kNBw; ++nb)
          dst[16 * nb] = (uint16_t)f32_to_bf16_bits(o[rb][nb][e] * inv);
      } else {
        float* dst = a.ws_acc + (po.st_base + (size_t)row * po.st_stride) * kDV + 64 * w + j;
#pragma unroll
        for (int nb = 0; nb < kNBw; ++nb) dst[16 * nb] = o[rb][nb][e];
      }
    }
  }
#if MLA_PHASE_TIMING
  MLA_STAMP(ph_end);
  MLA_PHASE_ADD(kPhEpilogue, ph_vote, ph_end);
  ph[kPhPieces] += 1;
  if (lane == 0 && blockIdx.x + gridDim.x * blockIdx.y < 256) {
    unsigned long long* row = mla_phase_cycles[(blockIdx.x + gridDim.x * blockIdx.y) * kWaves + w];
    for (int c = 0; c < kPhKernel; ++c) atomicAdd(row + c, (unsigned long long)ph[c]);
  }
#endif
}

// Fixed splits: workgroup (rg, b, split) takes split `split` of request b,
// cut at multiples of 32 tokens.
template <bool kBlockUniform>
__global__ __launch_bounds__(kThreads, 1) void mla_decode_kernel(const MlaArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kLdsBytes];
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
  mla_piece<kBlockUniform>(a, smem, b, blockIdx.x, S, seg_start, seg_end, po);
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

// Workgroup (w, rg): share w of row group rg. Every workgroup first plans
// the launch itself from seq_lens (no separate plan launch): the tile counts'
// inclusive prefix sums over chunks of the batch (one chunk per thread, a
// scan in P buffer 1, which the first piece does not touch before its
// second barrier) give T, the working share count n = min(nshare, T), the
// share's tiles and its first request. Workgroup (0, 0) also writes the
// request prefix sums pre[b] (b = 0..B), pre[B] = T and pre[B + 1] = n for
// the merge kernel, before any workgroup can return.
template <bool kBlockUniform>
__global__ __launch_bounds__(kThreads, 1) void mla_decode_balanced_kernel(const MlaArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kLdsBytes];
  const int w = blockIdx.x, rg = blockIdx.y;
  const int s_cap = a.max_blocks * a.block_size;
  auto tiles_of = [&](int b) -> uint64_t {
    const int S = min(max(a.seq_lens[b], 0), s_cap);
    return (uint64_t)((S + kTile - 1) / kTile);
  };
  uint64_t* const part = reinterpret_cast<uint64_t*>(smem + kDepth * kTileBytes + kPBytes);
  const int tid = threadIdx.x;
  const int per = (a.B + kThreads - 1) / kThreads;
  const int b0 = min(tid * per, a.B), b1 = min(b0 + per, a.B);
  uint64_t sum = 0;
  for (int b = b0; b < b1; ++b) sum += tiles_of(b);
  part[tid] = sum;
  __syncthreads();
  for (int off = 1; off < kThreads; off <<= 1) {  // inclusive scan of the chunk sums
    const uint64_t v = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  const uint64_t T = part[kThreads - 1];
  const int n = (int)(T < (uint64_t)a.nshare ? T : (uint64_t)a.nshare);
  if (w == 0 && rg == 0) {
    uint64_t run = part[tid] - sum;
    for (int b = b0; b < b1; ++b) {
      a.pre[b] = run;
      run += tiles_of(b);
    }
    if (tid == 0) {
      a.pre[a.B] = T;
      a.pre[a.B + 1] = (uint64_t)n;
    }
  }
  if (w >= n) return;
  const uint64_t t0 = share_start(T, w, n), t_end = share_start(T, w + 1, n);
  // The share's first request: the first b whose tiles end past t0 (the
  // chunk first, by bisection of the chunk prefix sums, then within it).
  int lo = 0, hi = kThreads - 1;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (part[mid] > t0) hi = mid; else lo = mid + 1;
  }
  uint64_t p0 = lo > 0 ? part[lo - 1] : 0;  // tiles before request b
  int b = lo * per;
  for (uint64_t nt = tiles_of(b); p0 + nt <= t0; nt = tiles_of(b)) {
    p0 += nt;
    ++b;
  }
#if MLA_PHASE_TIMING
  const uint64_t k_t0 = __builtin_amdgcn_s_memtime(), k_r0 = __builtin_amdgcn_s_memrealtime();
#endif
  for (uint64_t t = t0; t < t_end; ++b) {
    const uint64_t p1 = p0 + tiles_of(b);
    if (p1 <= t) {  // a request with no tiles
      p0 = p1;
      continue;
    }
    const uint64_t t1 = p1 < t_end ? p1 : t_end;
    const int S = min(max(a.seq_lens[b], 0), s_cap);
    PieceOut po;
    po.direct = t == p0 && t1 == p1;
    po.st_base = (size_t)(2 * w + (t == t0 ? 0 : 1)) * a.R;
    po.st_stride = 1;
    mla_piece<kBlockUniform>(a, smem, b, rg, S, (int)(t - p0) * kTile,
                             min(S, (int)(t1 - p0) * kTile), po);
    t = t1;
    p0 = p1;
  }
#if MLA_PHASE_TIMING
  const uint64_t k_t1 = __builtin_amdgcn_s_memtime(), k_r1 = __builtin_amdgcn_s_memrealtime();
  if ((threadIdx.x & 63) == 0 && w + gridDim.x * rg < 256) {
    unsigned long long* row = mla_phase_cycles[(w + gridDim.x * rg) * kWaves + (threadIdx.x >> 6)];
    atomicAdd(row + kPhKernel, (unsigned long long)(k_t1 - k_t0));
    atomicAdd(row + kPhKernelRealtime, (unsigned long long)(k_r1 - k_r0));
  }
#endif
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
    hipLaunchKernelGGL(mla::mla_decode_kernel<true>, grid, dim3(mla::kThreads), 0, stream, a);
  else
    hipLaunchKernelGGL(mla::mla_decode_kernel<false>, grid, dim3(mla::kThreads), 0, stream, a);
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
  return align16(states * (mla::kDV + 2) * sizeof(float)) + (size_t)(B + 2) * 8;
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
  a.pre = reinterpret_cast<uint64_t*>(ws + align16(states * (mla::kDV + 2) * sizeof(float)));
  a.nshare = n;
  const unsigned rg = (unsigned)((a.R + mla::kRowsPerGroup - 1) / mla::kRowsPerGroup);
  if (block_size % mla::kTile == 0)
    hipLaunchKernelGGL(mla::mla_decode_balanced_kernel<true>, dim3(n, rg), dim3(mla::kThreads), 0,
                       stream, a);
  else
    hipLaunchKernelGGL(mla::mla_decode_balanced_kernel<false>, dim3(n, rg), dim3(mla::kThreads), 0,
                       stream, a);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  const size_t rows = (size_t)B * a.R;
  hipLaunchKernelGGL(mla::mla_decode_balanced_merge_kernel, dim3((unsigned)((rows + 3) / 4)),
                     dim3(256), 0, stream, a);
  return hipGetLastError();
}


#if MLA_PHASE_TIMING
// Profiling build only (not part of include/mla_decode.h): copies the phase
// cycle table (2048 x kPhCols uint64, see mla_phase_cycles) to host memory,
// or with reset != 0 zeroes it first. Returns a hipError_t code.
extern "C" __attribute__((visibility("default"))) int mla_decode_phase_table(void* host,
                                                                            int reset) {
  static unsigned long long zero[2048][mla::kPhCols];
  if (reset)
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(mla::mla_phase_cycles), zero, sizeof(zero));
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(mla::mla_phase_cycles), sizeof(zero));
}
#endif
