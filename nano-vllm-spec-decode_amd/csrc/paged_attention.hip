// Paged attention for decode / speculative verify (replaces flash_attn_with_kvcache,
// nanovllm/layers/attention.py:71-78) and for varlen prefill / mixed prefill+decode (replaces
// flash_attn_varlen_func, attention.py:64-70). One kernel family serves both.
//
// Work decomposition. A work item is (sequence, query group, KV head):
//   * query group: P consecutive query positions of one sequence; with g = Hq/Hkv heads sharing the KV
//     head, the group holds P*g "rows" (row r = position r/g, head r%g) — GQA head-group sharing: the
//     KV stream is read once for all g query heads.
//   * the item's keys are cut into 32-key tiles; tile t belongs to residue t % 8. One wave streams the
//     tiles of one residue in increasing order with an online softmax, giving a partial (max, sum, O) per
//     row; the 8 residue partials are merged in residue order 0..7 with a fixed fma chain. This reduction
//     tree depends on nothing but the key positions, so a row's output is bitwise independent of the
//     batch size, of the number of query rows per sequence and of whether the step is a decode, a verify
//     or a mixed step.
// How residues map to hardware is chosen per launch from the amount of work, without changing the
// arithmetic: with many items one 8-wave workgroup owns an item's 8 residues and merges them in LDS
// (no workspace, no second kernel); with few items each workgroup owns 1, 2 or 4 residues, writes their
// partials to the workspace, and attn_combine runs the same merge.
//
// Per tile a wave computes, with bf16 MFMA 16x16x32 (rows in 16-row tiles, RT of them):
//   S^T[16 keys x 16 rows] = K[16 x 128] . Q^T      A = K straight from HBM into registers (16 B per
//                                                    lane, 64 contiguous bytes per key row per load),
//                                                    B = Q in registers for the whole item
//                                                    (three or four row tiles: read from LDS)
//   O^T[16 d x 16 rows]   += V^T[16 x 32] . P^T      A = V^T read transposed from LDS with
//                                                    ds_read_b64_tr_b16, B = P straight from S^T's
//                                                    accumulators (the key order inside the 32-key
//                                                    k-step is permuted identically for P and V^T)
// V is loaded 16 B per lane into registers, each lane fetching the chunk that its LDS store places,
// XOR-swizzled, so that the transposed reads are bank-conflict free. The next tile's V loads are issued
// as soon as the current V is in LDS and its K loads as soon as S^T is computed, so 16 KB per wave are
// in flight while the MFMAs and the softmax run; at <= 256 VGPRs two waves share a SIMD.
#include <math.h>

#include <algorithm>
#include <climits>
#include <type_traits>

#include "prefill_attention.h"
#include "sd_common.h"
#include "../../include/sd_attn.h"

namespace sd {
namespace {

constexpr int kD = 128;                        // head_dim (Qwen3)
constexpr int kTile = 32;                      // keys per wave step
constexpr int kResidues = 8;                   // tile t belongs to residue t % 8
constexpr int kVBuf = kTile * kD * 2;          // one 32-key V tile in LDS: 8 KB per wave
constexpr int kObRow = kD + 4;                 // fp32 row stride of the merge buffer (bank padding)
constexpr int kMaxRows = 64;                   // 16-row tiles: at most 4
constexpr int kMaxBlocks = 2048;               // block-table entries staged in LDS per item (64 K keys at block
                                               // size 32, 512 K at 256)
constexpr int kMlBytes = kResidues * kMaxRows * 2 * 4;
constexpr int kMergeRows = 32;                 // rows merged in LDS per pass (two row tiles)
constexpr int kObBytes = kResidues * kMergeRows * kObRow * 4;

// LDS of a workgroup with `waves` waves: the V buffers, one per wave, or two with the two-tiles-ahead
// pipeline (`deep`; when the workgroup merges all eight residues the same bytes then hold every residue's
// O), the merge's (max, sum) table, and the item's block ids.
constexpr int stage_bytes(int waves, bool deep = false) {
  return waves == kResidues ? ((deep ? 2 : 1) * waves * kVBuf > kObBytes ? (deep ? 2 : 1) * waves * kVBuf : kObBytes)
                            : (deep ? 2 : 1) * waves * kVBuf;
}
constexpr int ml_bytes(int waves) { return waves == kResidues ? kMlBytes : 0; }
constexpr int lds_bytes(int waves, bool deep = false) {
  return stage_bytes(waves, deep) + ml_bytes(waves) + kMaxBlocks * 4;
}
// Three and four row tiles read Q from LDS at every tile instead of holding it in registers (16 registers per
// row tile), so that three fit in 256 registers and run two waves per SIMD. Q rows of 256 B past the block
// ids, the 16-byte chunk c of row r at c ^ (r % 16): the 16 lanes of a read take 16 different chunks.
// The two-tiles-ahead pipeline holds two tiles' K in registers and reads Q from LDS too, whatever RT.
constexpr bool q_in_lds(int rt, bool deep = false) { return deep || rt >= 3; }
constexpr int q_lds_bytes(int rt, bool deep = false) { return q_in_lds(rt, deep) ? rt * 16 * kD * 2 : 0; }
constexpr int q_lds_offset(int waves, bool deep = false) { return lds_bytes(waves, deep); }
constexpr int lds_bytes_rt(int waves, int rt, bool deep = false) {
  return lds_bytes(waves, deep) + q_lds_bytes(rt, deep);
}
static_assert(lds_bytes_rt(kResidues, 3, true) <= 160 * 1024, "eight waves with three row tiles fit the LDS");

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
// Cache-policy operand of global_load_lds: the non-temporal bit (the policy kv_load's non-temporal loads get).
constexpr int kCpolNT = 2;

struct Params {
  const uint16_t* q;
  int64_t q_stride;            // elements between consecutive query tokens (head stride = kD)
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_stride, v_stride;  // elements between consecutive key tokens / cache slots
  const int32_t* block_tables;
  int32_t table_width;
  int32_t block_size;
  int64_t num_blocks;
  const int32_t* context_lens;  // decode
  const int32_t* seq_order;     // decode: item i's sequence is seq_order[i / groups_per_seq] (null: i / groups)
  const int32_t* stream_flag;   // decode: nonzero -> non-temporal K / V loads (null: non-temporal)
  const int32_t* cu_q;          // varlen
  const int32_t* cu_k;          // varlen
  const int32_t* work;          // varlen: (sequence, group) pairs
  const int32_t* work_count;    // varlen: number of valid pairs
  int32_t n;                    // decode: queries per sequence
  int32_t groups_per_seq;       // decode: ceil(n / P)
  int32_t total_q;              // tokens in q
  int64_t total_k;              // varlen without block table: rows in k / v
  int32_t Hq, Hkv, g, P;
  int32_t rows_alloc;           // rows per (item, head, residue) partial
  float scale_log2;             // softmax scale * log2(e)
  uint16_t* out;
  int64_t out_stride;
  float* part_o;                // [item][Hkv][kResidues][rows_alloc][kD]
  float* part_ml;               // [item][Hkv][kResidues][rows_alloc][2] = (max, sum)
  int32_t wave_slots;           // workgroups the GPU runs at once (one per CU): the head rotation period
};

struct Item {
  int32_t seq, q_start, Lq, Lk, p0, np, kmax;
  bool valid;
};

template <bool kVarlen>
__device__ __forceinline__ Item describe(const Params& p, int item) {
  Item it;
  it.valid = false;
  int grp;
  if (kVarlen) {
    if (item >= *p.work_count) return it;
    it.seq = p.work[2 * item];
    grp = p.work[2 * item + 1];
    it.q_start = p.cu_q[it.seq];
    it.Lq = p.cu_q[it.seq + 1] - it.q_start;
    const int32_t k0 = p.cu_k[it.seq];
    it.Lk = p.cu_k[it.seq + 1] - k0;
    if (it.q_start < 0 || it.Lq < 0 || it.q_start + it.Lq > p.total_q || it.Lk < 0) return it;
    if (!p.block_tables && (k0 < 0 || (int64_t)k0 + it.Lk > p.total_k)) return it;
  } else {
    it.seq = p.seq_order ? p.seq_order[item / p.groups_per_seq] : item / p.groups_per_seq;
    if (it.seq < 0 || (int64_t)it.seq * p.n >= p.total_q) return it;  // an order entry out of range
    grp = item % p.groups_per_seq;
    it.q_start = it.seq * p.n;
    it.Lq = p.n;
    it.Lk = p.context_lens[it.seq];
    if (it.Lk < 0) it.Lk = 0;
  }
  if (p.block_tables && (int64_t)it.Lk > (int64_t)p.table_width * p.block_size)
    it.Lk = p.table_width * p.block_size;  // never index past the table row
  it.p0 = grp * p.P;
  it.np = min(p.P, it.Lq - it.p0);
  if (it.np <= 0) return it;
  it.kmax = min(max(it.Lk - it.Lq + it.p0 + it.np, 0), it.Lk);
  it.valid = true;
  return it;
}

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Max / sum over the four lanes l, l^16, l^32, l^48 (one row of a 16x16 accumulator tile).
__device__ __forceinline__ float quad_max(float x) {
  uint32_t a = __builtin_bit_cast(uint32_t, x), b = a;
  swap16(a, b);
  x = fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
  a = __builtin_bit_cast(uint32_t, x);
  b = a;
  swap32(a, b);
  return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}
__device__ __forceinline__ float quad_sum(float x) {
  uint32_t a = __builtin_bit_cast(uint32_t, x), b = a;
  swap16(a, b);
  x = __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
  a = __builtin_bit_cast(uint32_t, x);
  b = a;
  swap32(a, b);
  return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}

// A K / V load of the residue kernel. kStream: the non-temporal cache policy, for decode / verify calls
// whose contexts are balanced (B=64, k=4, ctx 4096: 185 -> 177 us). It costs where a launch ends in a
// latency-bound tail: decode over unbalanced contexts (lognormal, median 600: 59 -> 63 us) and the varlen /
// mixed launch (config-5 layer 45 -> 49 us), which therefore keep the default policy (see decode_plan).
template <bool kStream, class T>
__device__ __forceinline__ T kv_load(const uint8_t* ptr) {
  if constexpr (kStream)
    return __builtin_nontemporal_load((const T*)ptr);
  else
    return *(const T*)ptr;
}

// The residue merge used by both the in-workgroup path and attn_combine: M = max_r m_r; then, residue by
// residue in order 0..7, L = fma(l_r, f_r, L) and O = fma(O_r, f_r, O) from 0 with f_r = 2^(m_r - M);
// out = O / L (0 when L == 0). Explicit fmas keep the rounding identical in both places.
__device__ __forceinline__ float merge_scale(float m_r, float M) {
  return exp2_fast(m_r - (M == -INFINITY ? 0.f : M));
}

// One (item, KV head h) with the workgroup's kWaves waves, owning residues bx*kWaves .. +kWaves-1; `lds`
// holds lds_bytes_rt(kWaves, RT, kDeep). kDeep: tiles stream two ahead of the math instead of one (V through
// global_load_lds), the same arithmetic in the same order. (kCaller only separates the instantiations made from different kernels: the
// host compilation pass rejects one instantiation reached from two kernels.)
template <int RT, bool kVarlen, bool kPaged, int kWaves, int kCaller = 0, bool kNT = false, bool kDeep = false>
__device__ __forceinline__ void attn_body(const Params& p, uint8_t* lds, int item, int h, int bx) {
  constexpr bool kMergeHere = kWaves == kResidues;
  constexpr int kStageBytes = stage_bytes(kWaves, kDeep);
  constexpr bool kQLds = q_in_lds(RT, kDeep);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int residue = bx * kWaves + wave;
  const int lane = tid % kWave;
  const int r16 = lane % 16;  // row (S^T / O^T column) or key (K operand row) owned by this lane
  const int grp = lane / 16;  // 16-lane group: which 8 k-elements / 4 accumulator rows
  int32_t* blk_ids = (int32_t*)(lds + kStageBytes + ml_bytes(kWaves));

  // The block-table row loads (the whole row, ids are range-checked before use) go out before the item's
  // lengths arrive: a decode item knows its sequence without a memory read, a varlen item from the first
  // word of its work-list entry (written by the plan, always a sequence of the call).
  constexpr int kBlkPerThread = (kMaxBlocks + kWaves * kWave - 1) / (kWaves * kWave);
  int32_t blk_pre[kBlkPerThread];
  const int nblk_row = min(p.table_width, kMaxBlocks);
  // This wave's first two tiles (tiles `residue` and residue + 8) lie in table entries first_bi and
  // second_bi; their ids are read with the row, as scalar loads, so that the tiles' K and V loads can go out
  // before the row reaches LDS.
  const int first_bi = kPaged ? residue * kTile / p.block_size : 0;
  const int second_bi = kPaged ? (residue + kResidues) * kTile / p.block_size : 0;
  int32_t first_blk = -1, second_blk = -1;
  if (kPaged) {
    int seq = 0;
    bool listed = true;
    if (kVarlen) {
      listed = item < *p.work_count;
      if (listed) seq = p.work[2 * item];
    } else {
      seq = p.seq_order ? p.seq_order[item / p.groups_per_seq] : item / p.groups_per_seq;
      if (seq < 0 || (int64_t)seq * p.n >= p.total_q) seq = 0;  // describe() drops such an item
    }
    // Every thread loads (an index past the row reads its last id, then replaced by -1): no divergent
    // loads, so the waits before the LDS stores below count only these loads.
#pragma unroll
    for (int i = 0; i < kBlkPerThread; ++i) {
      const int b = tid + i * kWaves * kWave;
      const int32_t id = p.block_tables[(int64_t)seq * p.table_width + min(b, nblk_row - 1)];
      blk_pre[i] = listed && b < nblk_row ? id : -1;
    }
    if (listed) {
      first_blk = p.block_tables[(int64_t)seq * p.table_width + min(first_bi, nblk_row - 1)];
      second_blk = p.block_tables[(int64_t)seq * p.table_width + min(second_bi, nblk_row - 1)];
    }
  }
  const Item it = describe<kVarlen>(p, item);
  if (!it.valid) {
    // The ids are read on this path too, so that the compiler keeps their loads ahead of the length
    // checks instead of sinking them behind describe()'s round trips.
    if constexpr (kPaged) {
#pragma unroll
      for (int i = 0; i < kBlkPerThread; ++i) asm volatile("" : : "v"(blk_pre[i]));
      asm volatile("" : : "s"(first_blk), "s"(second_blk));
    }
    return;
  }
  const int rows = it.np * p.g;
  const int kmax = it.kmax;
  const int end_tile = (kmax + kTile - 1) / kTile;

  // Per-row visible-key limit (bottom-right causal: query i sees Lk - Lq + i + 1 keys) and the Q operand
  // (B of S^T): lane holds row 16*rt + r16, d = 32*ks + 8*grp + e.
  int lim[RT];
  bf16x8 qv[kQLds ? 1 : RT][4];
  uint8_t* qlds = lds + q_lds_offset(kWaves, kDeep);
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = rt * 16 + r16;
    if (row < rows) {
      const int i = it.p0 + row / p.g;
      lim[rt] = min(max(it.Lk - it.Lq + i + 1, 0), kmax);
      if constexpr (!kQLds) {
        const int hq = h * p.g + row % p.g;
        const uint16_t* qp = p.q + (int64_t)(it.q_start + i) * p.q_stride + hq * kD + 8 * grp;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) qv[rt][ks] = *(const bf16x8*)(qp + 32 * ks);
      }
    } else {
      lim[rt] = kmax;  // padding row: Q = 0 keeps its scores finite; never written
      if constexpr (!kQLds) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) qv[rt][ks] = bf16x8{};
      }
    }
  }
  if constexpr (kQLds) {
    // Q rows into LDS, one 16-byte chunk per thread and step (padding rows zero).
    constexpr int kChunks = RT * 16 * 16;
    for (int ci = tid; ci < kChunks; ci += kWaves * kWave) {
      const int row = ci / 16, c = ci % 16;
      u32x4 v = {0, 0, 0, 0};
      if (row < rows) {
        const int i = it.p0 + row / p.g;
        const int hq = h * p.g + row % p.g;
        v = *(const u32x4*)(p.q + (int64_t)(it.q_start + i) * p.q_stride + hq * kD + 8 * c);
      }
      *(u32x4*)(qlds + row * 256 + 16 * (c ^ (row % 16))) = v;
    }
    __syncthreads();
  }
  // Q operand of row tile rt, k-step ks (B of S^T): from registers, or the lane's chunk 4 ks + grp of row
  // 16 rt + r16 in LDS.
  auto q_frag = [&](int rt, int ks) -> bf16x8 {
    if constexpr (kQLds)
      return *(const bf16x8*)(qlds + (rt * 16 + r16) * 256 + 16 * ((4 * ks + grp) ^ r16));
    else
      return qv[rt][ks];
  };

  float m[RT], l[RT];
  f32x4 o[8][RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m[rt] = -INFINITY;
    l[rt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt][rt] = f32x4{};
  }

  uint8_t* const vring = lds + wave * (kDeep ? 2 : 1) * kVBuf;  // this wave's V buffer(s)
  // V^T reads (ds_read_b64_tr_b16): source lane reads 4 d of key tl (+16 for the second half) at
  // d = 16*dt + 4*(lane%4): chunk 2*dt + (lane%4)/2, byte 8*(lane%2) inside it.
  // That chunk, (2 dt + (lane%4)/2) ^ 2 (tl%8), is 2 (dt ^ (tl%8)) + (lane%4)/2: one xor per read from two
  // lane constants (no per-d-tile offset registers).
  const int tl = 4 * grp + r16 / 4;
  const uint32_t vt_base = tl * 256 + 8 * (lane % 2) + 16 * ((lane % 4) / 2);
  const uint32_t vt_x = 32 * (tl % 8);
  auto vt_off = [&](int dt) { return vt_base + (vt_x ^ (32u * dt)); };

  // Tile addressing: K / V base of tile jt (wave-uniform byte pointers; keys past the item's end read the
  // tile's first key instead: finite data, masked out in the softmax). An invalid block id (bad table)
  // never faults: its K and V come from block 0 and every key of the tile is masked, its V zero-filled.
  struct TileSrc {
    const uint8_t* kb;
    const uint8_t* vb;
    int nvalid;
    bool ok;
  };
  const int64_t ksb = p.k_stride * 2, vsb = p.v_stride * 2;  // bytes per key
  auto tile_src = [&](int jt, int blk) {
    TileSrc ts;
    const int t0 = jt * kTile;
    ts.nvalid = min(kTile, kmax - t0);
    ts.ok = true;
    int64_t row0;
    if (kPaged) {
      ts.ok = blk >= 0 && blk < p.num_blocks;
      row0 = (int64_t)(ts.ok ? blk : 0) * p.block_size + t0 % p.block_size;
    } else {
      row0 = (int64_t)p.cu_k[it.seq] + t0;
    }
    ts.kb = (const uint8_t*)p.k + row0 * ksb + h * kD * 2;
    ts.vb = (const uint8_t*)p.v + row0 * vsb + h * kD * 2;
    return ts;
  };
  auto tile_blk = [&](int jt) {
    const int bi = jt * kTile / p.block_size;
    if constexpr (kPaged && kDeep) {
      // inline asm read (a compiler-visible LDS read would wait for the V loads writing LDS in flight); the
      // ids were stored before the workgroup's barrier
      if (bi >= nblk_row) return -1;
      int32_t id;
      const uint32_t a = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const int32_t*)(blk_ids + bi);
      asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(id) : "v"(a) : "memory");
      return id;
    } else {
      return kPaged ? (bi < nblk_row ? blk_ids[bi] : -1) : 0;
    }
  };
  // K of a tile into registers (A of S^T): key 16*kt + r16, d = 32*ks + 8*grp + e; 32-bit lane offsets.
  const uint32_t k_off0 = (uint32_t)(r16 * ksb) + 16 * grp;
  const uint32_t k_off1 = k_off0 + (uint32_t)(16 * ksb);
  auto load_k = [&](const TileSrc& ts, bf16x8 (&kr)[2][4]) {
    const uint32_t off0 = r16 < ts.nvalid ? k_off0 : 16 * grp;
    const uint32_t off1 = 16 + r16 < ts.nvalid ? k_off1 : 16 * grp;
    if constexpr (kDeep) {
      // inline asm loads: next to the V loads into LDS in flight, the compiler would wait for every load
      // before any use of the K registers; the step's own vmcnt wait covers them
      const uint64_t base = (uint64_t)(uintptr_t)ts.kb;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        asm volatile("global_load_dwordx4 %0, %1, %2 offset:%3" : "=v"(kr[0][ks]) : "v"(off0), "s"(base), "i"(64 * ks)
                     : "memory");
        asm volatile("global_load_dwordx4 %0, %1, %2 offset:%3" : "=v"(kr[1][ks]) : "v"(off1), "s"(base), "i"(64 * ks)
                     : "memory");
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        kr[0][ks] = kv_load<kNT, bf16x8>(ts.kb + off0 + 64 * ks);
        kr[1][ks] = kv_load<kNT, bf16x8>(ts.kb + off1 + 64 * ks);
      }
    }
  };
  // V of a tile straight into one of this wave's LDS buffers (global_load_lds: lane L's 16 bytes land at
  // the instruction's base + 16 L): lane loads key t = 4*qd + lane/16, chunk (lane%16) ^ 2*(t%8), so that
  // slot lane%16 of row-group qd holds it XOR-swizzled; t%8 only depends on the parity of qd. No registers
  // hold V on its way, which leaves room for a second tile's K: two tiles in flight per wave.
  const int vf_key = lane / 16;
  const int vf_slot = lane % 16;
  const uint32_t v_c0 = 16 * (vf_slot ^ (2 * vf_key)), v_c1 = 16 * (vf_slot ^ (2 * (4 + vf_key)));
  const uint32_t v_off0 = (uint32_t)(vf_key * vsb) + v_c0, v_off1 = (uint32_t)(vf_key * vsb) + v_c1;
  auto dma_v = [&](const TileSrc& ts, uint8_t* vb) {
#pragma unroll
    for (int qd = 0; qd < 8; ++qd) {
      const bool valid = 4 * qd + vf_key < ts.nvalid;
      // a wave-uniform base plus a 32-bit lane offset (the scalar-base addressing form)
      const uint32_t off = valid ? (uint32_t)(4 * qd * vsb) + ((qd % 2) ? v_off1 : v_off0) : ((qd % 2) ? v_c1 : v_c0);
      __builtin_amdgcn_global_load_lds((const void*)(ts.vb + off), (lds_void*)(vb + 1024 * qd), 16, 0,
                                       kNT ? kCpolNT : 0);
    }
  };
  // The classic path: V as 16-byte register loads to the same lanes and slots, stored to the wave's first
  // buffer once the previous tile's V^T has been read.
  auto load_v = [&](const TileSrc& ts, u32x4 (&vs)[8]) {
#pragma unroll
    for (int qd = 0; qd < 8; ++qd) {
      const bool valid = 4 * qd + vf_key < ts.nvalid;
      const uint32_t off = (qd % 2) ? (valid ? v_off1 : v_c1) : (valid ? v_off0 : v_c0);
      vs[qd] = kv_load<kNT, u32x4>(ts.vb + (valid ? (int64_t)(4 * qd) * vsb : 0) + off);
    }
  };
  auto store_v = [&](const u32x4 (&vs)[8], bool ok, uint8_t* vb) {
#pragma unroll
    for (int qd = 0; qd < 8; ++qd) *(u32x4*)(vb + 1024 * qd + 16 * lane) = ok ? vs[qd] : u32x4{0, 0, 0, 0};
  };
  // A tile whose block id is invalid: its V (read from block 0) is replaced by zeros.
  auto zero_v = [&](uint8_t* vb) {
#pragma unroll
    for (int qd = 0; qd < 8; ++qd) *(u32x4*)(vb + 1024 * qd + 16 * lane) = u32x4{0, 0, 0, 0};
  };
  // V^T operand of d-tile dt (16 d x 32 keys) from V buffer vbuf: two transposed reads.
  auto read_vt = [&](const uint8_t* vbuf, int dt) {
    const uint32_t off = vt_off(dt);
    const v4i16 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)(vbuf + off));
    const v4i16 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4i16*)(vbuf + off + 16 * 256));
    const short e8 __attribute__((ext_vector_type(8))) = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    return __builtin_bit_cast(bf16x8, e8);
  };

  // V^T reads of the deep path: inline asm (the compiler would otherwise wait for every V load in flight
  // before reading any buffer), four d-tiles at a time, their results passed through one lgkmcnt(0).
  auto vt_frags4 = [&](const uint8_t* vbuf, int dt0, bf16x8 (&vt)[4]) {
    const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint8_t*)vbuf;
    u32x2 lo[4], hi[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      lo[d] = ds_read_tr16<0>(base + vt_off(dt0 + d));
      hi[d] = ds_read_tr16<16 * 256>(base + vt_off(dt0 + d));
    }
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(lo[0]), "+v"(lo[1]), "+v"(lo[2]), "+v"(lo[3]), "+v"(hi[0]), "+v"(hi[1]), "+v"(hi[2]),
                   "+v"(hi[3])
                 :
                 : "memory");
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const u32x4 w = {lo[d][0], lo[d][1], hi[d][0], hi[d][1]};
      vt[d] = __builtin_bit_cast(bf16x8, w);
    }
  };
  // One tile: S^T from the K registers, then (registers free) the next tile's K loads, then the online
  // softmax and O^T += V^T P^T.
  auto compute = [&](int jt, bool tile_ok, bf16x8 (&kr)[2][4], const uint8_t* vbuf, bool has_next,
                     const TileSrc& next) {
    const int t0 = jt * kTile;
    // S^T of row tile rt into s[.][rt] (or s[.][0] when the row tiles are interleaved).
    constexpr bool kInterleave = kQLds;  // three or four row tiles: S^T of one row tile live at a time
    f32x4 s[2][kInterleave ? 1 : RT];
    auto scores = [&](int rt, int slot) {
      s[0][slot] = s[1][slot] = f32x4{};
      if constexpr (kDeep) {
        // inline asm reads (a compiler-visible LDS read would wait for the V loads writing LDS in flight)
        bf16x8 qf[4];
        const uint32_t qa = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint8_t*)qlds +
                            (rt * 16 + r16) * 256;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) qf[ks] = ds_read_b128(qa + 16 * ((4 * ks + grp) ^ r16));
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(qf[0]), "+v"(qf[1]), "+v"(qf[2]), "+v"(qf[3]) : : "memory");
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          s[0][slot] = mfma16(kr[0][ks], qf[ks], s[0][slot]);
          s[1][slot] = mfma16(kr[1][ks], qf[ks], s[1][slot]);
        }
      } else {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const bf16x8 qf = q_frag(rt, ks);
          s[0][slot] = mfma16(kr[0][ks], qf, s[0][slot]);
          s[1][slot] = mfma16(kr[1][ks], qf, s[1][slot]);
        }
      }
    };
    if constexpr (!kInterleave) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) scores(rt, rt);
      if (has_next) load_k(next, kr);
    }
    bf16x8 pb[RT];
    const int tok0 = t0 + 4 * grp;  // keys of this lane: tok0 + (e%4) + 16*(e/4)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int slot = kInterleave ? 0 : rt;
      if constexpr (kInterleave) {
        scores(rt, 0);
        if (rt == RT - 1 && has_next) load_k(next, kr);
      }
      const int lim_e = (tile_ok ? lim[rt] : t0) - tok0;
      float x[8];
      float mx = -INFINITY;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x[e] = (e % 4) + 16 * (e / 4) < lim_e ? s[e / 4][slot][e % 4] * p.scale_log2 : -INFINITY;
        mx = fmaxf(mx, x[e]);
      }
      mx = quad_max(mx);
      const float m_new = fmaxf(m[rt], mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = exp2_fast(m[rt] - m_use);
      float sum = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x[e] = exp2_fast(x[e] - m_use);
        sum += x[e];
      }
      sum = quad_sum(sum);
      l[rt] = l[rt] * alpha + sum;
      m[rt] = m_new;
      if (!__all(alpha == 1.f)) {
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[dt][rt] *= alpha;
      }
      u32x4 w;
      w[0] = cvt_bf16x2(x[0], x[1]);
      w[1] = cvt_bf16x2(x[2], x[3]);
      w[2] = cvt_bf16x2(x[4], x[5]);
      w[3] = cvt_bf16x2(x[6], x[7]);
      pb[rt] = __builtin_bit_cast(bf16x8, w);
    }
    if constexpr (kDeep) {
#pragma unroll
      for (int dt0 = 0; dt0 < 8; dt0 += 4) {
        bf16x8 vt[4];
        vt_frags4(vbuf, dt0, vt);
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) o[dt0 + d][rt] = mfma16(vt[d], pb[rt], o[dt0 + d][rt]);
      }
    } else {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const bf16x8 vt = read_vt(vbuf, dt);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) o[dt][rt] = mfma16(vt, pb[rt], o[dt][rt]);
      }
    }
  };

  const int nt = residue < end_tile ? (end_tile - 1 - residue) / kResidues + 1 : 0;  // this wave's tiles
  if constexpr (!kDeep) {
    // One tile ahead: while tile j is computed, tile j+8's V is in flight (registers) and its K goes out as
    // soon as S^T has freed the K registers. The loop body issues its loads unconditionally and the last
    // tile is peeled: with a conditional load in the body the compiler's wait counts must cover the path
    // without it and would wait for the next tile's V before this tile's S^T.
    bf16x8 kreg[2][4];
    u32x4 vstage[8];
    int j = residue;
    bool cur_ok = true;
    {
      // The first tile from first_blk. Paged, a wave without tiles loads tile 0 of block 0 and never uses
      // it: loads on every path keep the waits before the LDS stores below exact.
      const bool has_tile = j < end_tile;
      const int blk0 = kPaged && has_tile && first_bi < nblk_row ? first_blk : -1;
      const TileSrc ts = tile_src(has_tile ? j : 0, __builtin_amdgcn_readfirstlane(blk0));
      if (kPaged || has_tile) {
        load_v(ts, vstage);
        load_k(ts, kreg);
      }
      cur_ok = ts.ok;
    }
    // The item's block ids in LDS for the later tiles (all kMaxBlocks entries, -1 past the row).
    if (kPaged) {
      static_assert(kBlkPerThread * kWaves * kWave == kMaxBlocks, "one id per thread and step");
#pragma unroll
      for (int i = 0; i < kBlkPerThread; ++i) blk_ids[tid + i * kWaves * kWave] = blk_pre[i];
      __syncthreads();
    }
    while (j + kResidues < end_tile) {
      const int blk_next = tile_blk(j + kResidues);
      lds_wave_fence();                  // previous tile's V^T reads (and the block id read) are complete
      store_v(vstage, cur_ok, vring);    // waits for this tile's V registers
      const TileSrc next = tile_src(j + kResidues, __builtin_amdgcn_readfirstlane(blk_next));
      load_v(next, vstage);              // next tile's V in flight during this tile's math
      __builtin_amdgcn_sched_barrier(0);  // keep those loads ahead of the S^T MFMAs
      lds_wave_fence();                  // the tile is in LDS before any lane reads it
      compute(j, cur_ok, kreg, vring, true, next);
      cur_ok = next.ok;
      j += kResidues;
    }
    if (j < end_tile) {
      lds_wave_fence();
      store_v(vstage, cur_ok, vring);
      lds_wave_fence();
      compute(j, cur_ok, kreg, vring, false, TileSrc{});
    }
  } else {
    // Two tiles ahead: while tile i is computed, tile i+1's K (registers) and V (LDS, global_load_lds) are in
    // flight, and tile i+2's loads go out as soon as tile i frees their registers (K, after S^T) and buffer
    // (V, after its V^T reads). K of even and odd tiles alternates between two register sets and V between
    // the two buffers, so the second set costs the registers that staged V in the classic path. No load
    // goes past the wave's last tile (the wave would wait for its round trip before the merge).
    uint8_t* const vb0 = vring;
    uint8_t* const vb1 = vring + kVBuf;
    bf16x8 ka[2][4], kb[2][4];
    bool ok0 = true, ok1 = true;
    // Past the wave's last tile a step still issues its sixteen loads (static counts: the compiler's waits for K
    // stay exact with two copies of the step), from one L2-hot 1 KB piece: the first row of block 0 of this
    // head, the same for every such load; never used.
    TileSrc dummy{};
    dummy.kb = (const uint8_t*)p.k + h * kD * 2;
    dummy.vb = (const uint8_t*)p.v + h * kD * 2;
    dummy.nvalid = 0;
    dummy.ok = true;
    TileSrc t0 = dummy, t1 = dummy;
    {
      const int blk0 = kPaged && nt > 0 && first_bi < nblk_row ? first_blk : -1;
      const int blk1 = kPaged && nt > 1 && second_bi < nblk_row ? second_blk : -1;
      if (nt > 0) t0 = tile_src(residue, __builtin_amdgcn_readfirstlane(blk0));
      if (nt > 1) t1 = tile_src(residue + kResidues, __builtin_amdgcn_readfirstlane(blk1));
      if (kPaged || nt > 0) {  // K into registers now; V (into LDS) after the block ids' barrier below
        load_k(t0, ka);
        load_k(t1, kb);
      }
      ok0 = t0.ok;
      ok1 = t1.ok;
    }
    if (kPaged) {
      static_assert(kBlkPerThread * kWaves * kWave == kMaxBlocks, "one id per thread and step");
#pragma unroll
      for (int i = 0; i < kBlkPerThread; ++i) blk_ids[tid + i * kWaves * kWave] = blk_pre[i];
      __syncthreads();
    }
    if (kPaged || nt > 0) {
      dma_v(t0, vb0);
      dma_v(t1, vb1);
    }
    // Step i: wait for tile i, compute it when it is one of the wave's tiles, and send tile i+2's loads (or the
    // stand-ins) into the registers and buffer it frees.
    // Straight-line (no branch around the math, so the compiler's waits for K stay exact): a step past the
    // wave's last tile computes a tile whose keys are all masked and whose V is zero, which leaves the row's
    // max, sum and O bitwise as they are.
    auto step = [&](int i, bf16x8 (&kr)[2][4], uint8_t* vb, bool& ok) {
      const int jt = residue + kResidues * i;
      TileSrc next = dummy;
      if (i + 2 < nt) next = tile_src(jt + 2 * kResidues, __builtin_amdgcn_readfirstlane(tile_blk(jt + 2 * kResidues)));
      const bool tile_ok = i < nt && ok;
      // Loads issued after tile i's V: tile i+1's K and V (16), except for tile 0, whose V goes out after the
      // barrier, behind tile 1's K: only tile 1's V (8) follows it.
      if (i == 0)
        asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
      if (!tile_ok) zero_v(vb);
      lds_wave_fence();
      compute(jt, tile_ok, kr, vb, true, next);
      lds_wave_fence();  // tile i's V^T reads are done: its buffer takes tile i+2
      dma_v(next, vb);
      ok = next.ok;
    };
    for (int i = 0; i < nt; i += 2) {
      step(i, ka, vb0, ok0);
      step(i + 1, kb, vb1, ok1);
    }
    // The last steps' K loads (never used) are still in flight: both register sets stay allocated until they
    // have landed, so that no other value takes those registers meanwhile.
    asm volatile("s_waitcnt vmcnt(0)"
                 :
                 : "v"(ka[0][0]), "v"(ka[0][1]), "v"(ka[0][2]), "v"(ka[0][3]), "v"(ka[1][0]), "v"(ka[1][1]),
                   "v"(ka[1][2]), "v"(ka[1][3]), "v"(kb[0][0]), "v"(kb[0][1]), "v"(kb[0][2]), "v"(kb[0][3]),
                   "v"(kb[1][0]), "v"(kb[1][1]), "v"(kb[1][2]), "v"(kb[1][3])
                 : "memory");
  }
  // every load has landed (also the unused ones): the V buffers may be reused
  if constexpr (kDeep) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  if constexpr (!kMergeHere) {
    // ---- write this residue's partial; attn_combine merges the eight ----
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int row = rt * 16 + r16;
      if (row >= rows) continue;
      const int64_t base = (((int64_t)item * p.Hkv + h) * kResidues + residue) * p.rows_alloc + row;
      float* po = p.part_o + base * kD + 4 * grp;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) *(f32x4*)(po + 16 * dt) = o[dt][rt];
      if (grp == 0) {
        p.part_ml[base * 2 + 0] = m[rt];
        p.part_ml[base * 2 + 1] = l[rt];
      }
    }
    return;
  } else {
    // ---- merge the eight residues in order: every wave parks its O in LDS, then each thread finishes
    // eight consecutive d of one row with the same fma chain as attn_combine; 32 rows per pass ----
    static_assert(RT * 16 <= kMaxRows, "row tiles");
    __syncthreads();  // all V^T (and Q) reads done: the stage bytes become the O store
    float* ml = (float*)(lds + kStageBytes);  // [residue][kMaxRows][2]
    float* ob = (float*)lds;                  // [residue][kMergeRows][kObRow]
    if (grp == 0) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        ml[(wave * kMaxRows + rt * 16 + r16) * 2 + 0] = m[rt];
        ml[(wave * kMaxRows + rt * 16 + r16) * 2 + 1] = l[rt];
      }
    }
    constexpr int kPassTiles = kMergeRows / 16;
#pragma unroll
    for (int pass = 0; pass * kPassTiles < RT; ++pass) {
      if (pass > 0) __syncthreads();  // the previous pass's reads of the O store are done
#pragma unroll
      for (int rt = pass * kPassTiles; rt < RT && rt < (pass + 1) * kPassTiles; ++rt) {
        if (rt * 16 + r16 >= rows) continue;  // padding rows are never read (LDS stores are the merge's cost)
        float* orow = ob + (wave * kMergeRows + (rt - pass * kPassTiles) * 16 + r16) * kObRow + 4 * grp;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) *(f32x4*)(orow + 16 * dt) = o[dt][rt];
      }
      __syncthreads();
      constexpr int kThreads = kWaves * kWave;
      const int row0 = pass * kMergeRows;
      const int pass_rows = min(RT * 16 - row0, kMergeRows);
      for (int e0 = tid * 8; e0 < pass_rows * kD; e0 += kThreads * 8) {
        const int prow = e0 / kD, d0 = e0 % kD;
        const int row = row0 + prow;
        if (row >= rows) continue;
        float M = -INFINITY;
#pragma unroll
        for (int r = 0; r < kResidues; ++r) M = fmaxf(M, ml[(r * kMaxRows + row) * 2]);
        float L = 0.f;
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r = 0; r < kResidues; ++r) {
          const float f = merge_scale(ml[(r * kMaxRows + row) * 2], M);
          L = __builtin_fmaf(ml[(r * kMaxRows + row) * 2 + 1], f, L);
          const float* src = ob + (r * kMergeRows + prow) * kObRow + d0;
          const f32x4 a = *(const f32x4*)src, b = *(const f32x4*)(src + 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            acc[e] = __builtin_fmaf(a[e], f, acc[e]);
            acc[4 + e] = __builtin_fmaf(b[e], f, acc[4 + e]);
          }
        }
        const int i = it.p0 + row / p.g;
        const int hq = h * p.g + row % p.g;
        u32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          w[e] = cvt_bf16x2(L == 0.f ? 0.f : acc[2 * e] / L, L == 0.f ? 0.f : acc[2 * e + 1] / L);
        *(u32x4*)(p.out + (int64_t)(it.q_start + i) * p.out_stride + hq * kD + d0) = w;
      }
    }
  }
}

// Workgroups are dispatched round-robin over the 8 XCDs in linear order (residue group fastest, then KV
// head, then item), so with 8 KV heads each XCD would run one head for the whole call. The heads' K/V
// segments of a key row do not stream equally fast (on the headline call two heads ran ~15 % slower,
// whichever XCD ran them), and that XCD's last workgroups then set the end of the call. The head is
// therefore rotated by one per batch of workgroups the GPU holds at once: an XCD runs one head at a
// time, a different one in each such batch (B=64 k=4: 193.7 -> 180.8 us).
__device__ __forceinline__ int rotated_head(const Params& p, int y, int z) {
  const int64_t linear = ((int64_t)z * gridDim.y + y) * gridDim.x;
  return (int)((y + linear / p.wave_slots) % p.Hkv);
}

// Two waves per SIMD (at most 256 registers a wave) up to three row tiles, whatever the workgroup size: the
// second argument is the minimum waves per SIMD. Four row tiles need more registers and run one wave a SIMD.
// Decode / verify with one or two row tiles streams two tiles ahead (kDeep): each residue wave walks the
// sequence's whole context in steps of 8 tiles, long enough for the deeper pipeline to pay (B=16, ctx 4096:
// 8-10 % faster); three row tiles would spill with it, and the varlen / mixed launch's short decode rows run
// faster with one tile ahead.
template <int RT, bool kVarlen>
constexpr bool deep_decode() { return !kVarlen && RT <= 2; }

template <int RT, bool kVarlen, bool kPaged, int kWaves>
__global__ __launch_bounds__(kWaves * kWave, RT <= 3 ? 2 : 1) void attn_fwd(Params p) {
  constexpr bool kDeep = deep_decode<RT, kVarlen>();
  __shared__ __attribute__((aligned(16))) uint8_t lds[lds_bytes_rt(kWaves, RT, kDeep)];
  const int h = rotated_head(p, blockIdx.y, blockIdx.z);
  if constexpr (kVarlen) {
    attn_body<RT, kVarlen, kPaged, kWaves>(p, lds, blockIdx.z, h, blockIdx.x);
  } else {
    // one uniform branch per workgroup between two copies of the body (load policy only)
    if (p.stream_flag == nullptr || *p.stream_flag != 0)
      attn_body<RT, kVarlen, kPaged, kWaves, 0, true, kDeep>(p, lds, blockIdx.z, h, blockIdx.x);
    else
      attn_body<RT, kVarlen, kPaged, kWaves, 0, false, kDeep>(p, lds, blockIdx.z, h, blockIdx.x);
  }
}

// Few (item, KV head) pairs (one-residue workgroups): the residue body with one wave keeps one 16 KB tile in
// flight and does each tile's math in one dependent chain, so such calls are bounded by latency. Here one
// wave streams the residue's tiles (three in registers, one ahead in a two-slot LDS ring, one barrier per
// tile) and four waves share the math: each takes one 16-row tile and a range of the 8 d-tiles of O (its
// rows' scores and softmax are computed by every wave that shares the row tile, identically). Rows and d
// columns are independent, so every output element goes through exactly the arithmetic of attn_body with
// one wave, in the same order: the partials written for attn_combine, and the results, are bitwise the
// same. The barriers wait for LDS only (prefill::block_sync), so the streaming wave's loads stay in flight
// across them.
constexpr int kStreamDepth = 3;                 // tiles in the streaming wave's registers
constexpr int kStreamMath = 4;                  // waves that do the math
constexpr int kStreamThreads = (kStreamMath + 1) * kWave;
constexpr int kSlotBytes = 2 * kVBuf;           // one K and one V tile
constexpr int kStreamLds = 2 * kSlotBytes + kMaxBlocks * 4;

template <int RT, bool kVarlen, bool kPaged>
__device__ __forceinline__ void stream_body(const Params& p, uint8_t* lds, int item, int h, int residue) {
  // Math wave c: row tile c / per_rt, d-tiles (c % per_rt) * DT .. +DT-1 (three row tiles: one each, wave 3
  // idle).
  constexpr int kPerRt = RT == 3 ? 1 : kStreamMath / RT;
  constexpr int DT = 8 / kPerRt;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const bool loader = wave == kStreamMath;
  const int lane = tid % kWave;
  const int r16 = lane % 16;
  const int grp = lane / 16;
  int32_t* blk_ids = (int32_t*)(lds + 2 * kSlotBytes);

  const Item it = describe<kVarlen>(p, item);
  if (!it.valid) return;
  const int rows = it.np * p.g;
  const int kmax = it.kmax;
  const int end_tile = (kmax + kTile - 1) / kTile;
  const int nblk_row = min(p.table_width, kMaxBlocks);
  if (kPaged) {
    for (int b = tid; b < nblk_row; b += kStreamThreads)
      blk_ids[b] = p.block_tables[(int64_t)it.seq * p.table_width + b];
    __syncthreads();
  }
  const int steps = residue < end_tile ? (end_tile - residue + kResidues - 1) / kResidues : 0;

  struct TileSrc {
    const uint8_t* kb;
    const uint8_t* vb;
    int nvalid;
    bool ok;
  };
  const int64_t ksb = p.k_stride * 2, vsb = p.v_stride * 2;
  // Tile jt's K / V base (past the last tile: the item's first tile, loaded and never read).
  auto tile_src = [&](int jt) {
    TileSrc ts;
    if (jt >= end_tile) jt = 0;
    const int t0 = jt * kTile;
    ts.nvalid = min(kTile, kmax - t0);
    ts.ok = true;
    int64_t row0;
    if (kPaged) {
      const int bi = t0 / p.block_size;
      const int blk = __builtin_amdgcn_readfirstlane(bi < nblk_row ? blk_ids[bi] : -1);
      ts.ok = blk >= 0 && blk < p.num_blocks;
      row0 = (int64_t)(ts.ok ? blk : 0) * p.block_size + t0 % p.block_size;
    } else {
      row0 = (int64_t)p.cu_k[it.seq] + t0;
    }
    ts.kb = (const uint8_t*)p.k + row0 * ksb + h * kD * 2;
    ts.vb = (const uint8_t*)p.v + row0 * vsb + h * kD * 2;
    return ts;
  };
  auto slot_k = [&](int s) { return lds + (s % 2) * kSlotBytes; };
  auto slot_v = [&](int s) { return lds + (s % 2) * kSlotBytes + kVBuf; };

  if (loader) {
    // ---- the streaming wave: K in the math waves' register layout (key 16*kt + r16, d = 32*ks + 8*grp + e;
    // keys past the tile's end read its first key), V in the residue body's LDS layout ----
    const uint32_t k_off0 = (uint32_t)(r16 * ksb) + 16 * grp;
    const uint32_t k_off1 = k_off0 + (uint32_t)(16 * ksb);
    const int vf_key = lane / 16;
    const int vf_slot = lane % 16;
    const uint32_t v_c0 = 16 * (vf_slot ^ (2 * vf_key)), v_c1 = 16 * (vf_slot ^ (2 * (4 + vf_key)));
    const uint32_t v_off0 = (uint32_t)(vf_key * vsb) + v_c0, v_off1 = (uint32_t)(vf_key * vsb) + v_c1;
    struct Regs {
      u32x4 k[8], v[8];
      bool ok;
    };
    auto load = [&](int s, Regs& r) {
      const TileSrc ts = tile_src(residue + kResidues * s);
      const uint32_t off0 = r16 < ts.nvalid ? k_off0 : 16 * grp;
      const uint32_t off1 = 16 + r16 < ts.nvalid ? k_off1 : 16 * grp;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        r.k[ks] = *(const u32x4*)(ts.kb + off0 + 64 * ks);
        r.k[4 + ks] = *(const u32x4*)(ts.kb + off1 + 64 * ks);
      }
#pragma unroll
      for (int qd = 0; qd < 8; ++qd) {
        const bool valid = 4 * qd + vf_key < ts.nvalid;
        const uint32_t off = (qd % 2) ? (valid ? v_off1 : v_c1) : (valid ? v_off0 : v_c0);
        r.v[qd] = *(const u32x4*)(ts.vb + (valid ? (int64_t)(4 * qd) * vsb : 0) + off);
      }
      r.ok = ts.ok;
    };
    auto store = [&](int s, const Regs& r) {
      uint8_t* kd = slot_k(s) + 16 * lane;
      uint8_t* vd = slot_v(s) + 16 * lane;
#pragma unroll
      for (int i = 0; i < 8; ++i) *(u32x4*)(kd + 1024 * i) = r.k[i];
#pragma unroll
      for (int qd = 0; qd < 8; ++qd) *(u32x4*)(vd + 1024 * qd) = r.ok ? r.v[qd] : u32x4{0, 0, 0, 0};
    };
    Regs ra, rb, rc;
    if (steps > 0) {
      load(0, ra);
      load(1, rb);
      load(2, rc);
      store(0, ra);
      load(3, ra);
    }
    prefill::block_sync();
    // Steps in threes so that every register set is static: tile s+1 is stored while the math waves work
    // on tile s, then tile s+4 is loaded into the freed set. Past the last step, loads and stores are of
    // valid addresses and never read.
    for (int s = 0; s < steps; s += kStreamDepth) {
      store(s + 1, rb);
      load(s + 4, rb);
      prefill::block_sync();
      if (s + 1 >= steps) break;
      store(s + 2, rc);
      load(s + 5, rc);
      prefill::block_sync();
      if (s + 2 >= steps) break;
      store(s + 3, ra);
      load(s + 6, ra);
      prefill::block_sync();
    }
    return;
  }

  // ---- a math wave: the residue body's arithmetic for one row tile and DT d-tiles ----
  const bool idle = wave >= RT * kPerRt;   // three row tiles: the fourth wave only keeps the barriers
  const int rt = idle ? 0 : wave / kPerRt;
  const int dt0 = (wave % kPerRt) * DT;
  const int row = rt * 16 + r16;
  int lim;
  bf16x8 qv[4];
  if (row < rows) {
    const int i = it.p0 + row / p.g;
    const int hq = h * p.g + row % p.g;
    lim = min(max(it.Lk - it.Lq + i + 1, 0), kmax);
    const uint16_t* qp = p.q + (int64_t)(it.q_start + i) * p.q_stride + hq * kD + 8 * grp;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qv[ks] = *(const bf16x8*)(qp + 32 * ks);
  } else {
    lim = kmax;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qv[ks] = bf16x8{};
  }
  float m = -INFINITY, l = 0.f;
  f32x4 o[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) o[d] = f32x4{};
  const int tl = 4 * grp + r16 / 4;
  uint32_t vt_off[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) {
    const int dt = dt0 + d;
    vt_off[d] = tl * 256 + 8 * (lane % 2) + 16 * (((2 * dt + (lane % 4) / 2) ^ (2 * (tl % 8))));
  }
  prefill::block_sync();  // the first tile is in slot 0

  for (int s = 0; s < steps; ++s) {
    if (!idle) {
      const int jt = residue + kResidues * s;
      const bool tile_ok = tile_src(jt).ok;
      const uint8_t* kt_lds = slot_k(s) + 16 * lane;
      const uint8_t* vbuf = slot_v(s);
      bf16x8 kr[2][4];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) kr[kt][ks] = *(const bf16x8*)(kt_lds + 1024 * (4 * kt + ks));
      const int t0 = jt * kTile;
      f32x4 sc[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        f32x4 acc = f32x4{};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) acc = mfma16(kr[kt][ks], qv[ks], acc);
        sc[kt] = acc;
      }
      const int tok0 = t0 + 4 * grp;
      const int lim_e = (tile_ok ? lim : t0) - tok0;
      float x[8];
      float mx = -INFINITY;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x[e] = (e % 4) + 16 * (e / 4) < lim_e ? sc[e / 4][e % 4] * p.scale_log2 : -INFINITY;
        mx = fmaxf(mx, x[e]);
      }
      mx = quad_max(mx);
      const float m_new = fmaxf(m, mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = exp2_fast(m - m_use);
      float sum = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x[e] = exp2_fast(x[e] - m_use);
        sum += x[e];
      }
      sum = quad_sum(sum);
      l = l * alpha + sum;
      m = m_new;
      if (!__all(alpha == 1.f)) {
#pragma unroll
        for (int d = 0; d < DT; ++d) o[d] *= alpha;
      }
      u32x4 w;
      w[0] = cvt_bf16x2(x[0], x[1]);
      w[1] = cvt_bf16x2(x[2], x[3]);
      w[2] = cvt_bf16x2(x[4], x[5]);
      w[3] = cvt_bf16x2(x[6], x[7]);
      const bf16x8 pb = __builtin_bit_cast(bf16x8, w);
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        const v4i16 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4i16*)(vbuf + vt_off[d]));
        const v4i16 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4i16*)(vbuf + vt_off[d] + 16 * 256));
        const short e8 __attribute__((ext_vector_type(8))) = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
        o[d] = mfma16(__builtin_bit_cast(bf16x8, e8), pb, o[d]);
      }
    }
    prefill::block_sync();  // this slot is free again; the next tile is in the other one
  }

  // ---- this residue's partial (this wave's rows and d range); attn_combine merges the eight ----
  if (idle || row >= rows) return;
  const int64_t base = (((int64_t)item * p.Hkv + h) * kResidues + residue) * p.rows_alloc + row;
  float* po = p.part_o + base * kD + 4 * grp;
#pragma unroll
  for (int d = 0; d < DT; ++d) *(f32x4*)(po + 16 * (dt0 + d)) = o[d];
  if (grp == 0 && dt0 == 0) {
    p.part_ml[base * 2 + 0] = m;
    p.part_ml[base * 2 + 1] = l;
  }
}

template <int RT, bool kVarlen, bool kPaged>
__global__ __launch_bounds__(kStreamThreads, 1) void attn_stream(Params p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kStreamLds];
  stream_body<RT, kVarlen, kPaged>(p, lds, blockIdx.z, rotated_head(p, blockIdx.y, blockIdx.z), blockIdx.x);
}

// A varlen call with long query runs: one launch for both work lists, so that the prefill q-blocks (MFMA
// and latency bound) and the decode / verify items (HBM bound) share the CUs. Slot x of the dispatch order
// takes the lists interleaved, two prefill q-blocks then one residue item (each list in its own order,
// longest first), then the rest of the longer list: the long prefill blocks start early without holding
// every CU while the decode rows wait, so HBM keeps streaming under the prefill math (config-5 layer 59 ->
// 49 us against the prefill list first). The q-blocks of sequences that see no key (the padding rows of a
// graph bucket: they only write zeros) come after both lists, so that they do not shift the interleave
// (they cost the 2048-token mixed layer 2 us, 45.5 against 43.5, in the interleave). A residue item runs all eight residues in the workgroup (merged in
// LDS, two row tiles). Slots past both lists exit; the grid has kMixedSlack spare slots for a partial last
// group.
constexpr int kMixedPre = 2, kMixedRes = 1;
constexpr int kMixedSlack = kMixedPre + kMixedRes - 2;
constexpr int kMixedLds = lds_bytes(kResidues) > prefill::kLdsBytes ? lds_bytes(kResidues) : prefill::kLdsBytes;
static_assert(prefill::kThreads == kResidues * kWave, "both halves use 512-thread workgroups");

template <bool kPaged, int kPreRowGroups, int kPreStageTiles>
__global__ __launch_bounds__(kResidues * kWave, 2) void mixed_fwd(Params p, PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kMixedLds];
  // KV head fastest along the grid, rotated by one per batch of resident workgroups (see rotated_head).
  const int h = (int)((blockIdx.x % a.Hkv + blockIdx.x / p.wave_slots) % a.Hkv);
  const int x = blockIdx.x / a.Hkv;
  // The plan's counts (each at most its grid share): np prefill q-blocks, the first npk of them from sequences
  // with keys (the rest see no key: a padded bucket's padding rows, which only write zeros), nr residue items.
  const int np = a.work_count[0], npk = a.work_count[1], nr = *p.work_count;
  constexpr int G = kMixedPre + kMixedRes;
  const int groups = min((npk + kMixedPre - 1) / kMixedPre, (nr + kMixedRes - 1) / kMixedRes);
  int pre = -1, res = -1;
  if (x < groups * G) {
    const int j = x / G, s = x % G;
    if (s < kMixedPre) {
      if (j * kMixedPre + s < npk) pre = j * kMixedPre + s;
    } else {
      res = j * kMixedRes + s - kMixedPre;
    }
  } else {
    // then the rest of the longer list, and the zero-key q-blocks last, so that they shift nothing
    const int y = x - groups * G;
    const int rest_pre = max(npk - groups * kMixedPre, 0), rest_res = max(nr - groups * kMixedRes, 0);
    if (y < rest_pre)
      pre = groups * kMixedPre + y;
    else if (y < rest_pre + rest_res)
      res = groups * kMixedRes + y - rest_pre;
    else
      pre = npk + y - rest_pre - rest_res;
  }
  if (pre >= 0 && pre < np)
    prefill::prefill_body<kPaged, kPreRowGroups, kPreStageTiles>(a, lds, pre, h);
  else if (res >= 0 && res < nr)
    attn_body<2, true, kPaged, kResidues, 1>(p, lds, res, h, 0);
}

// Merges the eight residue partials of every row, in residue order, with the same fma chain as the
// in-workgroup merge. One wave per row; each lane owns two d values.
template <bool kVarlen>
__global__ __launch_bounds__(256) void attn_combine(Params p) {
  const int item = blockIdx.x;
  const int h = blockIdx.y;
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  // One row per wave, four rows per workgroup along z: every row's loads are in flight at once, and they
  // go out before the item's description arrives (row < rows_alloc, so they stay inside the partials; the
  // rows past the item's are not used).
  const int row = blockIdx.z * 4 + wave;
  const int64_t base0 = (((int64_t)item * p.Hkv + h) * kResidues) * p.rows_alloc + row;
  float ms[kResidues], ls[kResidues];
  float2 os[kResidues];
#pragma unroll
  for (int r = 0; r < kResidues; ++r) {
    const int64_t b = base0 + (int64_t)r * p.rows_alloc;
    const float2 mlv = *(const float2*)(p.part_ml + b * 2);
    ms[r] = mlv.x;
    ls[r] = mlv.y;
    os[r] = *(const float2*)(p.part_o + b * kD + 2 * lane);
  }
  const Item it = describe<kVarlen>(p, item);
  if (!it.valid) return;
  const int rows = it.np * p.g;
  if (row < rows) {
    float M = -INFINITY;
#pragma unroll
    for (int r = 0; r < kResidues; ++r) M = fmaxf(M, ms[r]);
    float L = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int r = 0; r < kResidues; ++r) {
      const float f = merge_scale(ms[r], M);
      L = __builtin_fmaf(ls[r], f, L);
      o0 = __builtin_fmaf(os[r].x, f, o0);
      o1 = __builtin_fmaf(os[r].y, f, o1);
    }
    const int i = it.p0 + row / p.g;
    const int hq = h * p.g + row % p.g;
    uint16_t* op = p.out + (int64_t)(it.q_start + i) * p.out_stride + hq * kD;
    const float r0 = L == 0.f ? 0.f : o0 / L;
    const float r1 = L == 0.f ? 0.f : o1 / L;
    *(uint32_t*)(op + 2 * lane) = cvt_bf16x2(r0, r1);
  }
}

// Varlen work lists. A sequence with 1..kResidueMaxQ queries contributes ceil(Lq / P_res) (sequence, group)
// items of the residue kernel; a longer one contributes ceil(Lq / P_pre) (sequence, q-block) items of the
// prefill kernel, its last q-block (the one that sees the most keys) first. With at most kPlanThreads
// sequences, the sequences are taken in decreasing order of key count (ties by index; a bitonic sort in
// LDS), so that the longest work items are dispatched first and the short ones fill the tail; with more,
// in index order. The prefill count is written twice: all q-blocks, then those of sequences with keys (the
// zero-key ones, sorted last, are dispatched after everything else). One 1024-thread workgroup: each pass takes 1024 sequences (wave prefix sums, then the wave
// totals). The order changes only which workgroup computes an item, never an item's arithmetic.
constexpr int kPlanThreads = 1024;
__device__ __forceinline__ int wave_inclusive_sum(int x, int lane) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_up(x, off, kWave);
    if (lane >= off) x += y;
  }
  return x;
}

// Ascending bitonic sort of keys[0, width) in LDS by the workgroup (width a power of two <= its size;
// the padding keys 0xFFFFFFFF sort last). Narrow sorts (few sequences) take fewer barrier stages.
__device__ __forceinline__ int sort_width(int n) {
  int w = 64;
  while (w < n) w <<= 1;
  return w;
}
__device__ __forceinline__ void bitonic_sort(uint32_t* keys, int width) {
  const int tid = threadIdx.x;
  for (int k = 2; k <= width; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      const int other = tid ^ j;
      if (tid < width && other > tid) {
        const uint32_t a = keys[tid], b = keys[other];
        if ((a > b) == ((tid & k) == 0)) {
          keys[tid] = b;
          keys[other] = a;
        }
      }
      __syncthreads();
    }
  }
}

__global__ __launch_bounds__(kPlanThreads) void varlen_plan(const int32_t* __restrict__ cu_q,
                                                            const int32_t* __restrict__ cu_k, int32_t num_seqs,
                                                            int32_t P_res, int32_t P_pre,
                                                            int32_t* __restrict__ work_res, int32_t* __restrict__ count_res,
                                                            int32_t max_res, int32_t* __restrict__ work_pre,
                                                            int32_t* __restrict__ count_pre, int32_t max_pre) {
  constexpr int kPlanWaves = kPlanThreads / kWave;
  static_assert(kPlanThreads == 1024, "sort keys hold a 10-bit sequence index");
  __shared__ int32_t wsum[3][kPlanWaves];
  __shared__ int32_t carry[3];
  __shared__ uint32_t keys[kPlanThreads];
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const bool sorted = num_seqs <= kPlanThreads;
  if (tid < 3) carry[tid] = 0;
  if (sorted) {
    // key = (2^20 - 1 - key tiles) << 10 | sequence: ascending keys = descending work, then index order.
    uint32_t key = 0xFFFFFFFFu;
    if (tid < num_seqs) {
      const int Lk = max(cu_k[tid + 1] - cu_k[tid], 0);
      const uint32_t tiles = min((uint32_t)(Lk + kTile - 1) / kTile, (1u << 20) - 1);
      key = (((1u << 20) - 1 - tiles) << 10) | (uint32_t)tid;
    }
    keys[tid] = key;
    __syncthreads();
    bitonic_sort(keys, sort_width(num_seqs));
  }
  __syncthreads();
  for (int base = 0; base < num_seqs; base += kPlanThreads) {
    const int idx = base + tid;
    const int s = sorted ? (int)(keys[tid] & 1023u) : idx;
    int Lq = 0, Lk = 0;
    if (idx < num_seqs) {
      Lq = max(cu_q[s + 1] - cu_q[s], 0);
      Lk = cu_k[s + 1] - cu_k[s];
    }
    const int nr = Lq > 0 && Lq <= kResidueMaxQ ? (Lq + P_res - 1) / P_res : 0;
    const int nq = Lq > kResidueMaxQ ? (Lq + P_pre - 1) / P_pre : 0;
    const int ir = wave_inclusive_sum(nr, lane);
    const int iq = wave_inclusive_sum(nq, lane);
    const int ik = wave_inclusive_sum(Lk > 0 ? nq : 0, lane);
    if (lane == kWave - 1) {
      wsum[0][wave] = ir;
      wsum[1][wave] = iq;
      wsum[2][wave] = ik;
    }
    __syncthreads();
    int offr = carry[0], offq = carry[1], totr = 0, totq = 0, totk = 0;
    for (int w = 0; w < kPlanWaves; ++w) {
      if (w < wave) {
        offr += wsum[0][w];
        offq += wsum[1][w];
      }
      totr += wsum[0][w];
      totq += wsum[1][w];
      totk += wsum[2][w];
    }
    const int start_r = offr + ir - nr, start_q = offq + iq - nq;
    for (int i = 0; i < nr; ++i) {
      if (start_r + i < max_res) {
        work_res[2 * (start_r + i)] = s;
        work_res[2 * (start_r + i) + 1] = i;
      }
    }
    for (int i = 0; i < nq; ++i) {
      if (start_q + i < max_pre) {
        work_pre[2 * (start_q + i)] = s;
        work_pre[2 * (start_q + i) + 1] = nq - 1 - i;
      }
    }
    __syncthreads();
    if (tid == 0) {
      carry[0] += totr;
      carry[1] += totq;
      carry[2] += totk;
    }
    __syncthreads();
  }
  if (tid == 0) {
    *count_res = min(carry[0], max_res);
    count_pre[0] = min(carry[1], max_pre);
    // q-blocks of sequences with keys: a prefix of the list when it is sorted by key count (zero-key ones
    // last); in index order they may sit anywhere, and all count as keyed
    count_pre[1] = sorted ? min(carry[2], max_pre) : count_pre[0];
  }
}

// Decode / verify order: the sequences by context length, longest first (ties by index), so that the
// longest (sequence, KV head) workgroups are dispatched first and short ones fill the tail; up to
// kPlanThreads sequences (more: index order). Any permutation gives the same results: only which workgroup
// computes an item changes.
// Also writes order[num_seqs], the load-policy flag of the attention calls that use the plan: 1
// (non-temporal K / V loads) when the contexts are balanced, longest at most twice the mean, so that the call
// stays bandwidth-bound to its end; 0 when a few long contexts would leave a latency-bound tail.
__global__ __launch_bounds__(kPlanThreads) void decode_plan(const int32_t* __restrict__ context_lens, int32_t num_seqs,
                                                            int32_t* __restrict__ order) {
  __shared__ uint32_t keys[kPlanThreads];
  __shared__ int64_t wsum[kPlanThreads / kWave];
  __shared__ int32_t wmax[kPlanThreads / kWave];
  const int tid = threadIdx.x;
  if (num_seqs > kPlanThreads) {
    for (int i = tid; i < num_seqs; i += kPlanThreads) order[i] = i;
    if (tid == 0) order[num_seqs] = 1;
    return;
  }
  uint32_t key = 0xFFFFFFFFu;
  int L = 0;
  if (tid < num_seqs) {
    L = max(context_lens[tid], 0);
    const uint32_t tiles = min((uint32_t)(L + kTile - 1) / kTile, (1u << 20) - 1);
    key = (((1u << 20) - 1 - tiles) << 10) | (uint32_t)tid;
  }
  keys[tid] = key;
  int64_t sum = L;
  int mx = L;
  for (int off = 32; off >= 1; off >>= 1) {
    sum += __shfl_xor(sum, off);
    mx = max(mx, __shfl_xor(mx, off));
  }
  if (tid % kWave == 0) {
    wsum[tid / kWave] = sum;
    wmax[tid / kWave] = mx;
  }
  __syncthreads();
  bitonic_sort(keys, sort_width(num_seqs));
  if (tid < num_seqs) order[tid] = (int32_t)(keys[tid] & 1023u);
  if (tid == 0) {
    int64_t total = 0;
    int longest = 0;
    for (int w = 0; w < kPlanThreads / kWave; ++w) {
      total += wsum[w];
      longest = max(longest, wmax[w]);
    }
    order[num_seqs] = (int64_t)longest * num_seqs <= 2 * total ? 1 : 0;
  }
}

constexpr float kLog2e = 1.4426950408889634f;

// The number of 8-wave workgroups the device that runs `stream` holds at once: one per CU.
int wave_slots(hipStream_t stream) { return cu_count(stream); }

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct Layout {
  size_t part_o, part_ml, work, count, work_pre, count_pre, order, total;
};

// Workspace: residue partials only when the merge runs in attn_combine (few items); for varlen, the two
// work lists and their counts.
Layout workspace_layout(int64_t items, int Hkv, int rows_alloc, bool partials, bool varlen, int64_t pre_items = 0,
                        int64_t order_len = 0) {
  Layout L;
  const int64_t cells = partials ? items * Hkv * kResidues * rows_alloc : 0;
  L.part_o = 0;
  L.part_ml = align256(L.part_o + (size_t)cells * kD * sizeof(float));
  L.work = align256(L.part_ml + (size_t)cells * 2 * sizeof(float));
  L.count = align256(L.work + (varlen ? (size_t)items * 2 * sizeof(int32_t) : 0));
  L.work_pre = align256(L.count + (varlen ? sizeof(int32_t) : 0));
  L.count_pre = align256(L.work_pre + (varlen ? (size_t)pre_items * 2 * sizeof(int32_t) : 0));
  L.order = align256(L.count_pre + (varlen ? 2 * sizeof(int32_t) : 0));  // all q-blocks, those with keys
  L.total = align256(L.order + (size_t)(order_len ? order_len + 1 : 0) * sizeof(int32_t));  // + load-policy flag
  return L;
}

// 16-row tiles per item and positions per query group for n queries and g heads per KV head: the
// smallest tile count that holds all n*g rows (at most 4 tiles = 64 rows; more positions make more
// groups).
void decode_shape(int n, int g, int* RT, int* P) {
  const int rows = n * g;
  if (rows <= kMaxRows) {
    *RT = (rows + 15) / 16;
    *P = n;
  } else {
    *RT = 4;
    *P = kMaxRows / g;
  }
}

// Varlen prefill / mixed: 2 row tiles (32 rows) per group.
constexpr int kVarlenRT = 2;
static_assert(kVarlenRT == 2, "mixed_fwd runs the residue body with two row tiles");

// Waves per workgroup: all eight residues in one workgroup (merge in LDS) when there are enough
// (item, head) pairs to fill the GPU and the per-wave state allows two waves per SIMD; otherwise fewer
// residues per workgroup and more workgroups, with the merge in attn_combine.
int residue_waves(int64_t items, int Hkv, int RT) {
  const int64_t pairs = items * Hkv;
  if (RT <= 3 && pairs >= 256) return 8;
  if (pairs >= 128) return 4;
  if (pairs >= 32) return 2;
  return 1;
}

int check_heads(const char* who, int Hq, int Hkv, int D) {
  if (D != kD) return fail(kUnsupported, "%s: head_dim %d not supported (only %d)", who, D, kD);
  if (Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0)
    return fail(kBadArgument, "%s: num_heads %d must be a positive multiple of num_kv_heads %d", who, Hq, Hkv);
  if (Hq / Hkv > 16 * kVarlenRT)
    return fail(kUnsupported, "%s: more than %d query heads per KV head", who, 16 * kVarlenRT);
  return kOk;
}

template <int RT, bool kVarlen, bool kPaged>
void launch_rt(int waves, dim3 items_grid, hipStream_t s, const Params& p) {
  const dim3 grid(kResidues / waves, items_grid.y, items_grid.z);
  switch (waves) {
    case 8: hipLaunchKernelGGL((attn_fwd<RT, kVarlen, kPaged, 8>), grid, dim3(8 * kWave), 0, s, p); break;
    case 4: hipLaunchKernelGGL((attn_fwd<RT, kVarlen, kPaged, 4>), grid, dim3(4 * kWave), 0, s, p); break;
    case 2: hipLaunchKernelGGL((attn_fwd<RT, kVarlen, kPaged, 2>), grid, dim3(2 * kWave), 0, s, p); break;
    default: hipLaunchKernelGGL((attn_stream<RT, kVarlen, kPaged>), grid, dim3(kStreamThreads), 0, s, p); break;
  }
}

// Four row tiles need more than 256 registers per wave, so they never run eight waves per workgroup.
template <int RT, bool kVarlen, bool kPaged>
void launch_rt_small(int waves, dim3 items_grid, hipStream_t s, const Params& p) {
  const dim3 grid(kResidues / waves, items_grid.y, items_grid.z);
  switch (waves) {
    case 4: hipLaunchKernelGGL((attn_fwd<RT, kVarlen, kPaged, 4>), grid, dim3(4 * kWave), 0, s, p); break;
    case 2: hipLaunchKernelGGL((attn_fwd<RT, kVarlen, kPaged, 2>), grid, dim3(2 * kWave), 0, s, p); break;
    default: hipLaunchKernelGGL((attn_stream<RT, kVarlen, kPaged>), grid, dim3(kStreamThreads), 0, s, p); break;
  }
}

template <bool kVarlen, bool kPaged>
void launch_fwd(int RT, int waves, dim3 grid, hipStream_t s, const Params& p) {
  switch (RT) {
    case 1: launch_rt<1, kVarlen, kPaged>(waves, grid, s, p); break;
    case 2: launch_rt<2, kVarlen, kPaged>(waves, grid, s, p); break;
    case 3: launch_rt<3, kVarlen, kPaged>(waves, grid, s, p); break;
    default: launch_rt_small<4, kVarlen, kPaged>(waves, grid, s, p); break;
  }
}

}  // namespace
}  // namespace sd

using namespace sd;

extern "C" size_t sd_paged_decode_workspace_size(int32_t num_seqs, int32_t num_query_tokens, int32_t num_heads,
                                                 int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                                 int32_t table_width) {
  if (num_seqs <= 0 || num_query_tokens <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads) return 0;
  (void)head_dim;
  (void)block_size;
  (void)table_width;
  int RT, P;
  decode_shape(num_query_tokens, num_heads / num_kv_heads, &RT, &P);
  const int64_t items = (int64_t)num_seqs * ((num_query_tokens + P - 1) / P);
  const bool partials = residue_waves(items, num_kv_heads, RT) < kResidues;
  return workspace_layout(items, num_kv_heads, RT * 16, partials, false, 0, num_seqs).total;
}

namespace {
int decode_run(const char* who, bool planned, const void* q, int64_t q_token_stride, const void* k_cache,
               const void* v_cache, int64_t num_blocks, int32_t block_size, const int32_t* context_lens,
               const int32_t* block_tables, int32_t table_width, int32_t num_seqs, int32_t num_query_tokens,
               int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, float scale, void* out,
               int64_t out_token_stride, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_heads(who, num_heads, num_kv_heads, head_dim);
  if (rc) return rc;
  if (num_seqs < 0 || num_query_tokens <= 0 || table_width <= 0 || num_blocks <= 0)
    return fail(kBadArgument, "%s: bad sizes (seqs %d, queries %d, table width %d, blocks %lld)", who, num_seqs,
                num_query_tokens, table_width, (long long)num_blocks);
  if (block_size <= 0 || block_size % kTile)
    return fail(kUnsupported, "%s: block_size %d must be a positive multiple of %d", who, block_size, kTile);
  if (table_width > kMaxBlocks)
    return fail(kUnsupported, "%s: table width %d exceeds %d blocks", who, table_width, kMaxBlocks);
  if (num_seqs == 0) return kOk;
  if (!q || !k_cache || !v_cache || !context_lens || !block_tables || !out)
    return fail(kBadArgument, "%s: null pointer", who);
  if (q_token_stride < (int64_t)num_heads * head_dim || out_token_stride < (int64_t)num_heads * head_dim)
    return fail(kBadArgument, "%s: token stride smaller than num_heads*head_dim", who);
  if (((uintptr_t)q | (uintptr_t)out | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16 || q_token_stride % 8 ||
      out_token_stride % 8)
    return fail(kUnsupported, "%s: q / out / caches must be 16-byte aligned with strides multiple of 8", who);
  const int g = num_heads / num_kv_heads;
  int RT, P;
  decode_shape(num_query_tokens, g, &RT, &P);
  const int groups = (num_query_tokens + P - 1) / P;
  const int64_t items = (int64_t)num_seqs * groups;
  if (items > 65535) return fail(kUnsupported, "%s: %lld work items exceed the grid limit", who, (long long)items);
  const int waves = residue_waves(items, num_kv_heads, RT);
  const bool partials = waves < kResidues;
  const Layout lay = workspace_layout(items, num_kv_heads, RT * 16, partials, false, 0, num_seqs);
  // The unplanned call needs the workspace only for partials; the planned one reads the order from it.
  const size_t need = planned ? lay.total : partials ? lay.order : 0;
  if (need && (!workspace || workspace_bytes < need))
    return fail(kWorkspaceTooSmall, "%s: workspace %zu B < %zu B", who, workspace_bytes, need);

  Params p{};
  p.wave_slots = wave_slots((hipStream_t)stream);
  p.q = (const uint16_t*)q;
  p.q_stride = q_token_stride;
  p.k = (const uint16_t*)k_cache;
  p.v = (const uint16_t*)v_cache;
  p.k_stride = p.v_stride = (int64_t)num_kv_heads * head_dim;
  p.block_tables = block_tables;
  p.table_width = table_width;
  p.block_size = block_size;
  p.num_blocks = num_blocks;
  p.context_lens = context_lens;
  p.n = num_query_tokens;
  p.groups_per_seq = groups;
  p.total_q = num_seqs * num_query_tokens;
  p.Hq = num_heads;
  p.Hkv = num_kv_heads;
  p.g = g;
  p.P = P;
  p.rows_alloc = RT * 16;
  p.scale_log2 = scale * kLog2e;
  p.out = (uint16_t*)out;
  p.out_stride = out_token_stride;
  p.part_o = partials ? (float*)((uint8_t*)workspace + lay.part_o) : nullptr;
  p.part_ml = partials ? (float*)((uint8_t*)workspace + lay.part_ml) : nullptr;
  p.seq_order = planned ? (const int32_t*)((uint8_t*)workspace + lay.order) : nullptr;
  p.stream_flag = planned ? p.seq_order + num_seqs : nullptr;

  hipStream_t s = (hipStream_t)stream;
  launch_fwd<false, true>(RT, waves, dim3(1, num_kv_heads, (unsigned)items), s, p);
  if ((rc = check_launch(who))) return rc;
  if (partials) {
    // Four rows a workgroup over the rows a query group can hold (P positions x g heads), not the row tiles'
    // padding: B=16, k=4 merges 20 of 32 rows.
    const int merge_rows = std::min(P * g, p.rows_alloc);
    hipLaunchKernelGGL((attn_combine<false>), dim3((unsigned)items, num_kv_heads, (unsigned)((merge_rows + 3) / 4)),
                       dim3(256), 0, s, p);
    if ((rc = check_launch(who))) return rc;
  }
  return kOk;
}
}  // namespace

extern "C" int sd_paged_decode(const void* q, int64_t q_token_stride, const void* k_cache, const void* v_cache,
                               int64_t num_blocks, int32_t block_size, const int32_t* context_lens,
                               const int32_t* block_tables, int32_t table_width, int32_t num_seqs,
                               int32_t num_query_tokens, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                               float scale, void* out, int64_t out_token_stride, void* workspace,
                               size_t workspace_bytes, void* stream) {
  return decode_run("sd_paged_decode", false, q, q_token_stride, k_cache, v_cache, num_blocks, block_size,
                    context_lens, block_tables, table_width, num_seqs, num_query_tokens, num_heads, num_kv_heads,
                    head_dim, scale, out, out_token_stride, workspace, workspace_bytes, stream);
}

extern "C" int sd_paged_decode_planned(const void* q, int64_t q_token_stride, const void* k_cache,
                                       const void* v_cache, int64_t num_blocks, int32_t block_size,
                                       const int32_t* context_lens, const int32_t* block_tables, int32_t table_width,
                                       int32_t num_seqs, int32_t num_query_tokens, int32_t num_heads,
                                       int32_t num_kv_heads, int32_t head_dim, float scale, void* out,
                                       int64_t out_token_stride, void* workspace, size_t workspace_bytes,
                                       void* stream) {
  return decode_run("sd_paged_decode_planned", true, q, q_token_stride, k_cache, v_cache, num_blocks, block_size,
                    context_lens, block_tables, table_width, num_seqs, num_query_tokens, num_heads, num_kv_heads,
                    head_dim, scale, out, out_token_stride, workspace, workspace_bytes, stream);
}

extern "C" int sd_paged_decode_plan(const int32_t* context_lens, int32_t num_seqs, int32_t num_query_tokens,
                                    int32_t num_heads, int32_t num_kv_heads, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  const char* who = "sd_paged_decode_plan";
  if (num_seqs < 0 || num_query_tokens <= 0 || num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads)
    return fail(kBadArgument, "%s: bad sizes", who);
  if (num_seqs == 0) return kOk;
  if (!context_lens) return fail(kBadArgument, "%s: null pointer", who);
  int RT, P;
  decode_shape(num_query_tokens, num_heads / num_kv_heads, &RT, &P);
  const int64_t items = (int64_t)num_seqs * ((num_query_tokens + P - 1) / P);
  const bool partials = residue_waves(items, num_kv_heads, RT) < kResidues;
  const Layout lay = workspace_layout(items, num_kv_heads, RT * 16, partials, false, 0, num_seqs);
  if (!workspace || workspace_bytes < lay.total)
    return fail(kWorkspaceTooSmall, "%s: workspace %zu B < %zu B", who, workspace_bytes, lay.total);
  hipLaunchKernelGGL(decode_plan, dim3(1), dim3(kPlanThreads), 0, (hipStream_t)stream, context_lens, num_seqs,
                     (int32_t*)((uint8_t*)workspace + lay.order));
  return check_launch(who);
}

namespace {
int varlen_positions(int g) { return max(1, 16 * kVarlenRT / g); }
// Upper bounds of the two work lists (the launch grids), from host-known sizes only.
int64_t varlen_items(int32_t num_seqs, int32_t total_q, int P) {
  const int64_t per_seq = (kResidueMaxQ + P - 1) / P;
  return std::min<int64_t>((int64_t)num_seqs * per_seq, (int64_t)(total_q + P - 1) / P + num_seqs);
}
int64_t prefill_items(int32_t num_seqs, int32_t total_q, int32_t max_seqlen_q, int P) {
  if (max_seqlen_q <= kResidueMaxQ) return 0;
  return (int64_t)(total_q + P - 1) / P + std::min<int64_t>(num_seqs, total_q / (kResidueMaxQ + 1));
}
// Rows per prefill q-block (one geometry for every call, so that a row's result never depends on the batch
// or the chunking around it). 256-row q-blocks stage each K / V tile once for twice the rows of 128-row
// q-blocks (whose 8 waves split the tiles between two parities), which halves the staging per FLOP; in
// exchange every wave walks all of the q-block's keys. At Qwen3-8B shapes: a 2048-token mixed step's
// attention 8 % and a 16 x 1024-query prefill 10 % faster, a single 2048-token prompt 26 % slower.
constexpr int kPrefillRows = kPrefillRowsLarge;
constexpr int kPrefillRowGroups = kPrefillRows / 32;
// Two tiles a stage (32 KB), both computed by every wave: half the barriers of one tile a stage, the same
// arithmetic in the same order (bitwise equal outputs); 16 x 1024-query prefill 2-3 % faster.
constexpr int kPrefillStageTiles = 2;
int prefill_positions(int g) { return kPrefillRows / g; }

// Launch shape and workspace layout of a varlen call; a function of the host-known sizes only, shared by
// the planning and the attention entry points.
struct VarlenShape {
  int g, P;
  int64_t items, pre_items;  // grid sizes (upper bounds) of the residue and prefill work lists
  int waves;
  bool partials;
  Layout lay;
};
VarlenShape varlen_shape(int32_t num_seqs, int32_t total_q, int32_t max_seqlen_q, int32_t Hq, int32_t Hkv) {
  VarlenShape v;
  v.g = Hq / Hkv;
  v.P = varlen_positions(v.g);
  v.items = varlen_items(num_seqs, total_q, v.P);
  v.pre_items = prefill_items(num_seqs, total_q, max_seqlen_q, prefill_positions(v.g));
  v.waves = residue_waves(v.items, Hkv, kVarlenRT);
  // With prefill items the call is one mixed_fwd launch, whose residue items always merge in LDS: no partials.
  v.partials = v.waves < kResidues && v.pre_items == 0;
  v.lay = workspace_layout(v.items, Hkv, 16 * kVarlenRT, v.partials, true, v.pre_items);
  return v;
}

int launch_plan(const int32_t* cu_q, const int32_t* cu_k, int32_t num_seqs, const VarlenShape& v, void* workspace,
                hipStream_t s) {
  hipLaunchKernelGGL(varlen_plan, dim3(1), dim3(kPlanThreads), 0, s, cu_q, cu_k, num_seqs, v.P, prefill_positions(v.g),
                     (int32_t*)((uint8_t*)workspace + v.lay.work), (int32_t*)((uint8_t*)workspace + v.lay.count),
                     (int32_t)v.items, (int32_t*)((uint8_t*)workspace + v.lay.work_pre),
                     (int32_t*)((uint8_t*)workspace + v.lay.count_pre), (int32_t)v.pre_items);
  return check_launch("sd_varlen_plan");
}
}  // namespace

extern "C" size_t sd_varlen_workspace_size(int32_t num_seqs, int32_t total_q, int32_t max_seqlen_k, int32_t num_heads,
                                           int32_t num_kv_heads, int32_t head_dim) {
  if (num_seqs <= 0 || total_q <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads) return 0;
  (void)head_dim;
  (void)max_seqlen_k;
  const int g = num_heads / num_kv_heads;
  const int P = varlen_positions(g);
  const int64_t items = varlen_items(num_seqs, total_q, P);
  // The larger of the two launch forms: residue items alone (partials when they are few), or with the most
  // prefill items any max_seqlen_q allows (no partials).
  const int64_t pre_items = g <= 16 * kVarlenRT ? prefill_items(num_seqs, total_q, INT_MAX, prefill_positions(g)) : 0;
  const bool partials = residue_waves(items, num_kv_heads, kVarlenRT) < kResidues;
  return std::max(workspace_layout(items, num_kv_heads, 16 * kVarlenRT, partials, true, 0).total,
                  workspace_layout(items, num_kv_heads, 16 * kVarlenRT, false, true, pre_items).total);
}

namespace {
int varlen_run(const char* who, bool planned, const void* q, int64_t q_token_stride, const void* k,
               int64_t k_token_stride, const void* v, int64_t v_token_stride, int64_t total_k, int64_t num_blocks,
               int32_t block_size, const int32_t* block_tables, int32_t table_width, const int32_t* cu_seqlens_q,
               const int32_t* cu_seqlens_k, int32_t num_seqs, int32_t total_q, int32_t max_seqlen_q,
               int32_t max_seqlen_k, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, float scale,
               void* out, int64_t out_token_stride, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_heads(who, num_heads, num_kv_heads, head_dim);
  if (rc) return rc;
  if (num_seqs < 0 || total_q < 0 || max_seqlen_q < 0 || max_seqlen_k < 0)
    return fail(kBadArgument, "%s: bad sizes", who);
  if (num_seqs == 0 || total_q == 0) return kOk;
  if (!q || !k || !v || !cu_seqlens_q || !cu_seqlens_k || !out) return fail(kBadArgument, "%s: null pointer", who);
  const bool paged = table_width > 0;
  if (paged) {
    if (!block_tables || num_blocks <= 0 || block_size <= 0 || block_size % kTile)
      return fail(kBadArgument, "%s: paged mode needs a block table, blocks and a block_size multiple of %d", who, kTile);
    if (k_token_stride != (int64_t)num_kv_heads * head_dim || v_token_stride != k_token_stride)
      return fail(kBadArgument, "%s: paged caches must have token stride num_kv_heads*head_dim", who);
    if (table_width > kMaxBlocks)
      return fail(kUnsupported, "%s: table width %d exceeds %d blocks", who, table_width, kMaxBlocks);
  } else if (k_token_stride < (int64_t)num_kv_heads * head_dim || v_token_stride < (int64_t)num_kv_heads * head_dim) {
    return fail(kBadArgument, "%s: k / v token stride smaller than num_kv_heads*head_dim", who);
  }
  if (q_token_stride < (int64_t)num_heads * head_dim || out_token_stride < (int64_t)num_heads * head_dim)
    return fail(kBadArgument, "%s: token stride smaller than num_heads*head_dim", who);
  if (((uintptr_t)q | (uintptr_t)out | (uintptr_t)k | (uintptr_t)v) % 16 || q_token_stride % 8 ||
      out_token_stride % 8 || k_token_stride % 8 || v_token_stride % 8)
    return fail(kUnsupported, "%s: q / out / k / v must be 16-byte aligned with strides multiple of 8", who);
  const VarlenShape vs = varlen_shape(num_seqs, total_q, max_seqlen_q, num_heads, num_kv_heads);
  const int g = vs.g, P = vs.P, waves = vs.waves;
  const int64_t items = vs.items, pre_items = vs.pre_items;
  const bool partials = vs.partials;
  const Layout& lay = vs.lay;
  if (items > 65535) return fail(kUnsupported, "%s: %lld work items exceed the grid limit", who, (long long)items);
  if ((pre_items + items + kMixedSlack) * num_kv_heads > INT_MAX / 2)
    return fail(kUnsupported, "%s: too many prefill blocks", who);
  if (!workspace || workspace_bytes < lay.total)
    return fail(kWorkspaceTooSmall, "%s: workspace %zu B < %zu B", who, workspace_bytes, lay.total);

  Params p{};
  p.wave_slots = wave_slots((hipStream_t)stream);
  p.q = (const uint16_t*)q;
  p.q_stride = q_token_stride;
  p.k = (const uint16_t*)k;
  p.v = (const uint16_t*)v;
  p.k_stride = k_token_stride;
  p.v_stride = v_token_stride;
  p.block_tables = paged ? block_tables : nullptr;
  p.table_width = table_width;
  p.block_size = paged ? block_size : 1;
  p.num_blocks = num_blocks;
  p.cu_q = cu_seqlens_q;
  p.cu_k = cu_seqlens_k;
  p.total_q = total_q;
  p.total_k = total_k;
  p.Hq = num_heads;
  p.Hkv = num_kv_heads;
  p.g = g;
  p.P = P;
  p.rows_alloc = 16 * kVarlenRT;
  p.scale_log2 = scale * kLog2e;
  p.out = (uint16_t*)out;
  p.out_stride = out_token_stride;
  p.part_o = partials ? (float*)((uint8_t*)workspace + lay.part_o) : nullptr;
  p.part_ml = partials ? (float*)((uint8_t*)workspace + lay.part_ml) : nullptr;
  int32_t* work = (int32_t*)((uint8_t*)workspace + lay.work);
  int32_t* count = (int32_t*)((uint8_t*)workspace + lay.count);
  p.work = work;
  p.work_count = count;

  int32_t* work_pre = (int32_t*)((uint8_t*)workspace + lay.work_pre);
  int32_t* count_pre = (int32_t*)((uint8_t*)workspace + lay.count_pre);

  hipStream_t s = (hipStream_t)stream;
  if (!planned && (rc = launch_plan(cu_seqlens_q, cu_seqlens_k, num_seqs, vs, workspace, s))) return rc;
  if (pre_items > 0) {
    PrefillArgs a{};
    a.q = (const uint16_t*)q;
    a.q_stride = q_token_stride;
    a.k = (const uint16_t*)k;
    a.v = (const uint16_t*)v;
    a.k_stride = k_token_stride;
    a.v_stride = v_token_stride;
    a.block_tables = paged ? block_tables : nullptr;
    a.table_width = table_width;
    a.block_size = paged ? block_size : 1;
    a.tile_shift = -1;
    if (paged && ((block_size / kTile) & (block_size / kTile - 1)) == 0)
      a.tile_shift = __builtin_ctz((unsigned)(block_size / kTile));
    a.num_blocks = num_blocks;
    a.cu_q = cu_seqlens_q;
    a.cu_k = cu_seqlens_k;
    a.work = work_pre;
    a.work_count = count_pre;
    a.max_items = (int32_t)pre_items;
    a.total_q = total_q;
    a.total_k = total_k;
    a.Hkv = num_kv_heads;
    a.g = g;
    a.P = prefill_positions(g);
    a.scale_log2 = scale * kLog2e;
    a.out = (uint16_t*)out;
    a.out_stride = out_token_stride;
    // One launch for both lists; its residue items always merge in LDS (no partials, no combine). The KV
    // head varies fastest along the 1-D grid, so the work lists' order (longest first) is the dispatch order
    // across all heads; and as dispatch goes round-robin over the 8 XCDs, with 8 KV heads the q-blocks of
    // one head, which read the same K / V tiles, all run on one XCD and share its L2.
    const dim3 mgrid((unsigned)((pre_items + items + kMixedSlack) * num_kv_heads));
    if (paged)
      hipLaunchKernelGGL((mixed_fwd<true, kPrefillRowGroups, kPrefillStageTiles>), mgrid, dim3(kResidues * kWave), 0, s,
                         p, a);
    else
      hipLaunchKernelGGL((mixed_fwd<false, kPrefillRowGroups, kPrefillStageTiles>), mgrid, dim3(kResidues * kWave), 0,
                         s, p, a);
    return check_launch(who);
  }
  const dim3 grid(1, num_kv_heads, (unsigned)items);
  if (paged)
    launch_rt<kVarlenRT, true, true>(waves, grid, s, p);
  else
    launch_rt<kVarlenRT, true, false>(waves, grid, s, p);
  if ((rc = check_launch(who))) return rc;
  if (partials) {
    hipLaunchKernelGGL((attn_combine<true>), dim3((unsigned)items, num_kv_heads, (unsigned)(p.rows_alloc / 4)),
                       dim3(256), 0, s, p);
    if ((rc = check_launch(who))) return rc;
  }
  return kOk;
}
}  // namespace

extern "C" int sd_varlen_attention(const void* q, int64_t q_token_stride, const void* k, int64_t k_token_stride,
                                   const void* v, int64_t v_token_stride, int64_t total_k, int64_t num_blocks,
                                   int32_t block_size, const int32_t* block_tables, int32_t table_width,
                                   const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int32_t num_seqs,
                                   int32_t total_q, int32_t max_seqlen_q, int32_t max_seqlen_k, int32_t num_heads,
                                   int32_t num_kv_heads, int32_t head_dim, float scale, void* out,
                                   int64_t out_token_stride, void* workspace, size_t workspace_bytes, void* stream) {
  return varlen_run("sd_varlen_attention", false, q, q_token_stride, k, k_token_stride, v, v_token_stride, total_k,
                    num_blocks, block_size, block_tables, table_width, cu_seqlens_q, cu_seqlens_k, num_seqs, total_q,
                    max_seqlen_q, max_seqlen_k, num_heads, num_kv_heads, head_dim, scale, out, out_token_stride,
                    workspace, workspace_bytes, stream);
}

extern "C" int sd_varlen_attention_planned(const void* q, int64_t q_token_stride, const void* k,
                                           int64_t k_token_stride, const void* v, int64_t v_token_stride,
                                           int64_t total_k, int64_t num_blocks, int32_t block_size,
                                           const int32_t* block_tables, int32_t table_width,
                                           const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int32_t num_seqs,
                                           int32_t total_q, int32_t max_seqlen_q, int32_t max_seqlen_k,
                                           int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, float scale,
                                           void* out, int64_t out_token_stride, void* workspace,
                                           size_t workspace_bytes, void* stream) {
  return varlen_run("sd_varlen_attention_planned", true, q, q_token_stride, k, k_token_stride, v, v_token_stride,
                    total_k, num_blocks, block_size, block_tables, table_width, cu_seqlens_q, cu_seqlens_k, num_seqs,
                    total_q, max_seqlen_q, max_seqlen_k, num_heads, num_kv_heads, head_dim, scale, out,
                    out_token_stride, workspace, workspace_bytes, stream);
}

extern "C" int sd_varlen_plan(const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int32_t num_seqs,
                              int32_t total_q, int32_t max_seqlen_q, int32_t num_heads, int32_t num_kv_heads,
                              void* workspace, size_t workspace_bytes, void* stream) {
  const char* who = "sd_varlen_plan";
  if (num_seqs < 0 || total_q < 0 || max_seqlen_q < 0 || num_kv_heads <= 0 || num_heads <= 0 ||
      num_heads % num_kv_heads)
    return fail(kBadArgument, "%s: bad sizes", who);
  if (num_seqs == 0 || total_q == 0) return kOk;
  if (!cu_seqlens_q || !cu_seqlens_k) return fail(kBadArgument, "%s: null pointer", who);
  const VarlenShape vs = varlen_shape(num_seqs, total_q, max_seqlen_q, num_heads, num_kv_heads);
  if (vs.items > 65535) return fail(kUnsupported, "%s: %lld work items exceed the grid limit", who, (long long)vs.items);
  if (!workspace || workspace_bytes < vs.lay.total)
    return fail(kWorkspaceTooSmall, "%s: workspace %zu B < %zu B", who, workspace_bytes, vs.lay.total);
  return launch_plan(cu_seqlens_q, cu_seqlens_k, num_seqs, vs, workspace, (hipStream_t)stream);
}
