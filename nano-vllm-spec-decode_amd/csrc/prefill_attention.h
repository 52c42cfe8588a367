// Varlen attention for long query runs: the prefill chunks of a prefill or mixed prefill+decode step
// (replaces flash_attn_varlen_func for those sequences, nanovllm/layers/attention.py:64-70; sequences with
// at most kResidueMaxQ queries stay on the residue kernel of paged_attention.hip).
//
// Prefill is MFMA work (Q·K^T and P·V over many query rows per key), so the decomposition differs from the
// HBM-streaming decode kernel: one 8-wave workgroup owns a q-block of 128 or 256 rows (P query positions x g
// query heads of one KV head) and walks the keys in 32-key tiles shared through LDS by all its waves.
//   * 128 rows: wave w is row group rg = w % 4 (rows 32rg .. 32rg+31 of the block) of parity w / 4: it takes
//     the tiles t with t % 2 == parity, with its own online softmax; the two parity partials are merged at
//     the end (parity 0 then 1, fixed order). 256 rows: wave w is row group w and takes every tile.
//     Either way the reduction depends only on key positions, and a row's result is the same whichever
//     chunk, q-block or batch the row is computed in (for a given q-block size).
//   * A stage is one or two consecutive K and V tiles (16 or 32 KB; with two parities, one tile per parity).
//     Each lane loads its 16-byte pieces of it (2 or 4) into registers two stages ahead and writes them to
//     the LDS double buffer one stage ahead; one barrier per stage.
//     Register staging (rather than global_load_lds) keeps every wait count visible to the compiler.
//   * v_mfma_f32_32x32x16_bf16 for both products:
//       S^T[32 keys x 32 rows] = K . Q^T   A = K from LDS (ds_read_b128), B = Q in registers
//       O^T[32 d x 32 rows]   += V^T . P^T A = V^T from LDS (ds_read_b64_tr_b16), B = P straight from
//                                          S^T's accumulators (keys permuted identically in V^T)
//     A row's 32 scores of a tile sit in two lanes (l, l^32), so each row reduction is one lane swap.
//   * Masks are applied only on tiles that cross a row's causal limit. A row's reference maximum is
//     raised (and O, l rescaled) only when a tile's maximum exceeds it by more than 2^8 in the exp2
//     domain, so probabilities stay <= 256 and most tiles skip the rescale; the decision is the row's own.
// LDS layouts (16-byte chunks c of a 256-byte key row, XOR-swizzled so that both read patterns are
// bank-conflict free): K chunk c of key j at slot c ^ (j % 16); V chunk c of key j at slot c ^ 4*(j % 4).
#pragma once
#include <math.h>

#include "sd_common.h"

namespace sd {

// Sequences with at most this many queries in a varlen call take the residue kernel (the decode / verify
// arithmetic, bitwise equal to sd_paged_decode); longer query runs take the prefill kernel.
constexpr int kResidueMaxQ = 16;
// Rows (query position x query head of one KV head) per prefill q-block: 128 (the 8 waves as 4 row groups x
// 2 parities) or 256 (8 row groups, one parity).
constexpr int kPrefillRowsSmall = 128;
constexpr int kPrefillRowsLarge = 256;

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_stride;             // elements between consecutive query tokens (head stride 128)
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_stride, v_stride;   // elements between consecutive key tokens / cache slots
  const int32_t* block_tables;  // null: keys are rows cu_k[s] + j of k / v
  int32_t table_width;
  int32_t block_size;
  int32_t tile_shift;           // log2(block_size / 32) when that is a power of two, else -1
  int64_t num_blocks;
  const int32_t* cu_q;
  const int32_t* cu_k;
  const int32_t* work;          // (sequence, q-block) pairs written by varlen_plan
  const int32_t* work_count;
  int32_t max_items;            // grid size (upper bound of *work_count)
  int32_t total_q;
  int64_t total_k;
  int32_t Hkv, g, P;            // P = query positions per q-block (P * g <= the q-block's rows)
  float scale_log2;             // softmax scale * log2(e)
  uint16_t* out;
  int64_t out_stride;
};

}  // namespace sd

namespace sd {
namespace prefill {

constexpr int kD = 128;
constexpr int kTile = 32;                              // keys per tile
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kWave;               // 512
constexpr int kTileBytes = kTile * kD * 2;             // one K or V tile: 8 KB
constexpr int kStageBytesMax = 2 * 2 * kTileBytes;     // [parity][K, V] with two parities: 32 KB
constexpr int kStages = 2;                             // LDS stage buffers
constexpr int kMaxBlocks = 2048;                       // block-table entries staged in LDS
constexpr float kLazyLog2 = 8.f;                       // rescale threshold (exp2 domain)
constexpr int kLdsBytes = kStages * kStageBytesMax + kMaxBlocks * 4 + kWaves * 4;  // + per-wave flags
// The parity merge (two parities, four row groups) reuses the stage buffers and the block ids: O of the four
// parity-1 waves (64 fp32 per lane) + (m, l).
static_assert(4 * 64 * kWave * 4 + 4 * 2 * kWave * 4 <= kLdsBytes, "merge area");

typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// s_waitcnt through the builtin (not inline asm) so that the compiler's own wait insertion knows the loads
// are complete. gfx9 encoding: vmcnt in bits 3:0 (and 15:14), expcnt 6:4, lgkmcnt 11:8.
__device__ __forceinline__ void wait_vm_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

// All waves' LDS writes (plain stores, completed DMA) are visible after it.
__device__ __forceinline__ void block_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// One q-block (work item `widx`, KV head h) of kRowGroups * 32 rows with the workgroup's 512 threads; `lds`
// holds kLdsBytes. kRowGroups = 4: two parities; kRowGroups = 8: one parity, every wave takes every tile.
// A stage holds kStageTiles consecutive tiles; the wave of parity `par` computes tiles par, par + kParities,
// ... of each stage.
template <bool kPaged, int kRowGroups, int kStageTiles>
__device__ __forceinline__ void prefill_body(const PrefillArgs& p, uint8_t* lds, int widx, int h) {
  static_assert(kRowGroups == 4 || kRowGroups == 8, "q-blocks of 128 or 256 rows");
  constexpr int kParities = kWaves / kRowGroups;
  static_assert(kStageTiles % kParities == 0 && (kStageTiles == 1 || kStageTiles == 2), "tiles per stage");
  constexpr int kStageBytes = kStageTiles * 2 * kTileBytes;            // [tile][K, V]
  constexpr int kLoadsPerWave = kStageBytes / (kWaves * kWave * 16);  // 16-byte loads per lane per stage
  constexpr int kTileWaves = kWaves / kStageTiles;                     // waves loading one tile's K and V
  static_assert(kStageBytes <= kStageBytesMax && kLoadsPerWave * kWaves * 1024 == kStageBytes, "stage loads");
  if (widx >= *p.work_count) return;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid % kWave;
  const int rg = wave % kRowGroups;
  const int par = wave / kRowGroups;
  const int col = lane % 32;   // S^T / O^T column = this lane's row; K-operand key
  const int half = lane / 32;

  // ---- the work item (uniform over the workgroup) ----
  const int seq = p.work[2 * widx];
  const int qb = p.work[2 * widx + 1];
  const int q_start = p.cu_q[seq];
  const int Lq = p.cu_q[seq + 1] - q_start;
  const int k0 = p.cu_k[seq];
  int Lk = p.cu_k[seq + 1] - k0;
  if (q_start < 0 || Lq <= 0 || q_start + Lq > p.total_q || Lk < 0) return;
  if (!kPaged && (k0 < 0 || (int64_t)k0 + Lk > p.total_k)) return;
  if (kPaged && (int64_t)Lk > (int64_t)p.table_width * p.block_size) Lk = p.table_width * p.block_size;
  const int p0 = qb * p.P;
  const int np = min(p.P, Lq - p0);
  if (np <= 0) return;
  const int rows = np * p.g;
  const int kmax = min(max(Lk - Lq + p0 + np, 0), Lk);  // keys seen by the block's last position
  const int ntiles = (kmax + kTile - 1) / kTile;
  const int niter = (ntiles + kStageTiles - 1) / kStageTiles;

  // ---- block ids of the keys the block sees (to LDS below) and this lane's row: Q (B operand of S^T:
  // d = 16s + 8*half + e) and its visible-key limit; both loads in flight together ----
  int32_t* blk_ids = (int32_t*)(lds + kStages * kStageBytesMax);
  const int nblk_row = min(p.table_width, kMaxBlocks);
  const int nb_used = kPaged ? min((kmax + p.block_size - 1) / p.block_size, nblk_row) : 0;
  constexpr int kBlkPer = kMaxBlocks / kThreads;
  int32_t blk_pre[kBlkPer];
#pragma unroll
  for (int i = 0; i < kBlkPer; ++i) {
    const int b = tid + i * kThreads;
    blk_pre[i] = b < nb_used ? p.block_tables[(int64_t)seq * p.table_width + b] : 0;
  }
  const int row = rg * 32 + col;
  bf16x8 qv[8];
  int lim;
  if (row < rows) {
    const int i = p0 + row / p.g;
    const int hq = h * p.g + row % p.g;
    lim = min(max(Lk - Lq + i + 1, 0), kmax);
    const uint16_t* qp = p.q + (int64_t)(q_start + i) * p.q_stride + hq * kD + 8 * half;
#pragma unroll
    for (int s = 0; s < 8; ++s) qv[s] = *(const bf16x8*)(qp + 16 * s);
  } else {
    lim = kmax;  // padding row: Q = 0 keeps its scores finite; never written
#pragma unroll
    for (int s = 0; s < 8; ++s) qv[s] = bf16x8{};
  }
  wait_vm_all();  // Q and block ids in registers before any stage load is issued
  bool bad = false;
#pragma unroll
  for (int i = 0; i < kBlkPer; ++i) {
    const int b = tid + i * kThreads;
    if (b < nb_used) {
      blk_ids[b] = blk_pre[i];
      bad |= blk_pre[i] < 0 || blk_pre[i] >= p.num_blocks;
    }
  }
  static_assert(kBlkPer * kThreads == kMaxBlocks, "block ids per thread");
  int32_t* bad_flags = blk_ids + kMaxBlocks;  // one per wave: the wave staged an invalid block id
  const int wave_bad = __any(bad);
  if (lane == 0) bad_flags[wave] = wave_bad;
  // The wave's rows span positions first..last: limits grow with the position.
  const int first_row = rg * 32, last_row = min(rg * 32 + 31, rows - 1);
  const bool wave_active = first_row < rows;
  const int lim_lo = wave_active ? min(max(Lk - Lq + p0 + first_row / p.g + 1, 0), kmax) : 0;
  const int lim_hi = wave_active ? min(max(Lk - Lq + p0 + last_row / p.g + 1, 0), kmax) : 0;

  block_sync();  // block ids and flags visible
  // With valid ids only (the normal case) the tiles need no per-step check.
  int any_bad = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) any_bad |= bad_flags[w];
  any_bad = __builtin_amdgcn_readfirstlane(any_bad);

  // ---- stage loads: tiles 2*it and 2*it+1, K and V each, 1 KB per wave instruction ----
  const int64_t ksb = p.k_stride * 2, vsb = p.v_stride * 2;  // bytes per key row
  // Block-table index and in-block key offset of tile t (a tile never straddles two blocks).
  auto tile_index = [&](int t) { return p.tile_shift >= 0 ? t >> p.tile_shift : t * kTile / p.block_size; };
  auto tile_offset = [&](int t) {
    return p.tile_shift >= 0 ? (t & ((1 << p.tile_shift) - 1)) * kTile : (t * kTile) % p.block_size;
  };
  // The block id of tile t as read from LDS (0 past the last tile); read a step before it is needed, so
  // that the read completes under that step's compute.
  auto tile_block_raw = [&](int t) { return (!kPaged || t >= ntiles) ? 0 : blk_ids[tile_index(t)]; };
  // kTileWaves waves load each tile of a stage (K and V: 16 slots of 1 KB): wave w loads tile
  // w / kTileWaves of the stage, K in the first half of those waves and V in the second, kLoadsPerWave
  // consecutive slots each (two tiles a stage: slots 4*(w%2) .. +3; one: slots 2*(w%4) .. +1). Lane L of
  // slot j writes LDS bytes 16L.. of the slot, i.e. key 4j + L/16, physical chunk L%16, so it fetches the
  // logical chunk that the swizzle stores there. Stages past the last tile load valid rows that are never
  // stored, so that every stage issues the same loads (static wait counts).
  const int ld_par = wave / kTileWaves;
  const bool ld_v = (wave % kTileWaves) >= kTileWaves / 2;
  const int ld_slot0 = kLoadsPerWave * (wave % (kTileWaves / 2));
  const uint8_t* ld_src = (const uint8_t*)(ld_v ? p.v : p.k) + h * kD * 2;
  const int64_t ld_stride = ld_v ? vsb : ksb;
  uint32_t ld_off[kLoadsPerWave];   // byte offset of this lane's chunk inside key row `key`
  uint32_t ld_lane[kLoadsPerWave];  // paged: byte offset of that chunk from the tile's first key row
  int ld_key[kLoadsPerWave];
#pragma unroll
  for (int i = 0; i < kLoadsPerWave; ++i) {
    const int key = 4 * (ld_slot0 + i) + lane / 16;
    const int pc = lane % 16;
    ld_key[i] = key;
    ld_off[i] = 16 * (ld_v ? (pc ^ (4 * (key % 4))) : (pc ^ (key % 16)));
    ld_lane[i] = (uint32_t)(key * ld_stride) + ld_off[i];
  }
  // Paged: a wave-uniform base address (the tile's first key row) plus 32-bit lane offsets.
  auto load_stage = [&](int it, int blk_raw, u32x4 (&r)[kLoadsPerWave]) {
    const int t = kStageTiles * it + ld_par;
    if (kPaged) {
      const int blk = __builtin_amdgcn_readfirstlane(blk_raw);
      int64_t row0 = 0;  // cache slot of the tile's first key; block 0 past the end or for an invalid id
      if (t < ntiles && blk >= 0 && blk < p.num_blocks) row0 = (int64_t)blk * p.block_size + tile_offset(t);
      const uint8_t* base = ld_src + row0 * ld_stride;
#pragma unroll
      for (int i = 0; i < kLoadsPerWave; ++i) r[i] = *(const u32x4*)(base + ld_lane[i]);
    } else {
#pragma unroll
      for (int i = 0; i < kLoadsPerWave; ++i) {
        const int64_t krow = (int64_t)k0 + min(t * kTile + ld_key[i], max(Lk - 1, 0));
        r[i] = *(const u32x4*)(ld_src + krow * ld_stride + ld_off[i]);
      }
    }
  };
  auto stage_block = [&](int it) { return tile_block_raw(kStageTiles * it + ld_par); };
  auto store_stage = [&](int it, const u32x4 (&r)[kLoadsPerWave]) {
    uint8_t* dst = lds + (it % kStages) * kStageBytes + ld_par * 2 * kTileBytes + (ld_v ? kTileBytes : 0) +
                   ld_slot0 * 1024 + lane * 16;
#pragma unroll
    for (int i = 0; i < kLoadsPerWave; ++i) *(u32x4*)(dst + i * 1024) = r[i];
  };

  // ---- per-lane LDS read offsets ----
  // K operand of k-step s: key col, chunk 2s + half.
  const uint32_t k_row = col * 256;
  const uint32_t k_x = col % 16;
  // V^T operand (d-tile dt, key step kk): this lane supplies 4 d of key 16kk + 4*half + (lane%16)/4 (first
  // read; +8 keys for the second) at d0 = 32dt + 16*((lane/16)%2) + 4*(lane%4): chunk 4dt + cb, byte 8*(lane%2).
  const int v_key = 4 * half + (lane % 16) / 4;
  const uint32_t v_x = 4 * (v_key % 4);
  const uint32_t v_base = v_key * 256 + 8 * (lane % 2) + 16 * (2 * ((lane / 16) % 2) + (lane % 4) / 2);

  f32x16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x16{};
  float m_run = -INFINITY;  // running max of this lane's row (raw scores)
  float l_part = 0.f;       // this lane's share (16 of the 32 keys per tile) of the row's sum
  const float sl2 = p.scale_log2;

  // Per tile: the eight K operands are read together (one wait), the S^T MFMAs run, then the sixteen
  // V^T reads are issued before the softmax so that their latency hides behind it.
  auto compute = [&](const uint8_t* kt, const uint8_t* vt, int t, bool need_mask) {
    const uint32_t kt_addr = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint8_t*)kt + k_row;
    bf16x8 ka[8];
#pragma unroll
    for (int st = 0; st < 8; ++st) ka[st] = ds_read_b128(kt_addr + (((2 * st + half) ^ k_x) * 16));
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(ka[0]), "+v"(ka[1]), "+v"(ka[2]), "+v"(ka[3]), "+v"(ka[4]), "+v"(ka[5]), "+v"(ka[6]),
                   "+v"(ka[7])
                 :
                 : "memory");
    // The MFMA runs issue at raised wave priority: a wave with MFMAs ready goes first, so that the other
    // waves' softmax VALU work fills the matrix core's busy cycles (16 x 1024 prefill 5-7 % faster).
    f32x16 s = f32x16{};
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int st = 0; st < 8; ++st) s = mfma32(ka[st], qv[st], s);
    __builtin_amdgcn_s_setprio(0);
    const uint32_t vt_addr = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint8_t*)vt + v_base;
    u32x2 vr[4][4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const uint32_t a = vt_addr + (((4 * dt) ^ v_x) * 16);
      vr[dt][0] = ds_read_tr16<0>(a);      // keys 16kk + 4*half + j, kk = 0
      vr[dt][1] = ds_read_tr16<2048>(a);   //   + 8
      vr[dt][2] = ds_read_tr16<4096>(a);   // kk = 1
      vr[dt][3] = ds_read_tr16<6144>(a);
    }
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = s[r];
    if (need_mask) {
      const int kl = lim - (t * kTile + 4 * half);  // keys of register r: 8*(r/4) + r%4 (+ t0 + 4*half)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (8 * (r / 4) + r % 4 >= kl) x[r] = -INFINITY;
    }
    float mx = x[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, x[r]);
    uint32_t a0 = __builtin_bit_cast(uint32_t, mx), b0 = a0;
    swap32(a0, b0);
    mx = fmaxf(__builtin_bit_cast(float, a0), __builtin_bit_cast(float, b0));
    const bool raise = mx * sl2 > m_run * sl2 + kLazyLog2;
    if (!__all(!raise)) {
      const float alpha = raise ? exp2_fast((m_run - mx) * sl2) : 1.f;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
      l_part *= alpha;
      if (raise) m_run = mx;
    }
    const float mb = (m_run == -INFINITY ? 0.f : m_run) * sl2;
    float sum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      x[r] = exp2_fast(__builtin_fmaf(x[r], sl2, -mb));
      sum += x[r];
    }
    l_part += sum;
    bf16x8 pb[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      u32x4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = cvt_bf16x2(x[8 * kk + 2 * e], x[8 * kk + 2 * e + 1]);
      pb[kk] = __builtin_bit_cast(bf16x8, w);
    }
    // The V^T reads' results pass through the wait, so no MFMA can be scheduled before it.
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(vr[0][0]), "+v"(vr[0][1]), "+v"(vr[0][2]), "+v"(vr[0][3]), "+v"(vr[1][0]), "+v"(vr[1][1]),
                   "+v"(vr[1][2]), "+v"(vr[1][3]), "+v"(vr[2][0]), "+v"(vr[2][1]), "+v"(vr[2][2]), "+v"(vr[2][3]),
                   "+v"(vr[3][0]), "+v"(vr[3][1]), "+v"(vr[3][2]), "+v"(vr[3][3])
                 :
                 : "memory");
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const u32x4 w = {vr[dt][2 * kk][0], vr[dt][2 * kk][1], vr[dt][2 * kk + 1][0], vr[dt][2 * kk + 1][1]};
        o[dt] = mfma32(__builtin_bit_cast(bf16x8, w), pb[kk], o[dt]);
      }
    }
    __builtin_amdgcn_s_setprio(0);
  };

  // ---- pipeline: stage it in LDS, it+1 and it+2 in registers (ra / rb alternate) ----
  auto step = [&](int it) {
#pragma unroll
    for (int sub = 0; sub < kStageTiles; sub += kParities) {
      const int t = kStageTiles * it + sub + par;
      bool ok = true;
      if (kPaged && any_bad && t < ntiles) {
        const int blk = __builtin_amdgcn_readfirstlane(blk_ids[tile_index(t)]);
        ok = blk >= 0 && blk < p.num_blocks;
      }
      if (wave_active && t < ntiles && ok && t * kTile < lim_hi) {
        const uint8_t* kt = lds + (it % kStages) * kStageBytes + (sub + par) * 2 * kTileBytes;
        compute(kt, kt + kTileBytes, t, t * kTile + kTile > lim_lo);
      }
    }
  };
  u32x4 ra[kLoadsPerWave], rb[kLoadsPerWave];
  if (niter > 0) {
    load_stage(0, stage_block(0), ra);
    load_stage(1, stage_block(1), rb);
    store_stage(0, ra);
    load_stage(2, stage_block(2), ra);
    block_sync();  // stage 0 in LDS
  }
  // Straight-line halves (no conditional loads or stores) so that every wait count is static: stages
  // past the end are stored into a buffer that is never read again, and an odd last half-step computes
  // nothing (its tile index is >= ntiles).
  for (int it = 0; it < niter; it += 2) {
    const int blk3 = stage_block(it + 3);
    step(it);
    store_stage(it + 1, rb);  // buffer (it+1)%2 was last read in iteration it-1
    load_stage(it + 3, blk3, rb);
    block_sync();
    const int blk4 = stage_block(it + 4);
    step(it + 1);
    store_stage(it + 2, ra);
    load_stage(it + 4, blk4, ra);
    block_sync();
  }

  // ---- merge the two parities (parity 0 then 1) and write bf16 rows; one parity: normalize only ----
  uint32_t la = __builtin_bit_cast(uint32_t, l_part), lb = la;
  swap32(la, lb);
  const float l_row = __builtin_bit_cast(float, la) + __builtin_bit_cast(float, lb);
  float* mo = (float*)lds;                                    // [rg][64 values][64 lanes]
  float* mml = (float*)(lds + 4 * 64 * kWave * 4);            // [rg][m, l][64 lanes]
  float f0 = 1.f, f1 = 0.f, L = l_row;
  if constexpr (kParities == 2) {
    block_sync();  // every wave is done with the stage buffers
    if (par == 1) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) mo[(rg * 64 + dt * 16 + r) * kWave + lane] = o[dt][r];
      mml[(rg * 2 + 0) * kWave + lane] = m_run;
      mml[(rg * 2 + 1) * kWave + lane] = l_row;
    }
    block_sync();
  }
  wait_vm_all();  // the last two (unused) stage loads
  if (par == 1 || row >= rows) return;
  if constexpr (kParities == 2) {
    const float m1 = mml[(rg * 2 + 0) * kWave + lane];
    const float l1 = mml[(rg * 2 + 1) * kWave + lane];
    const float M = fmaxf(m_run, m1);
    const float Mu = M == -INFINITY ? 0.f : M;
    f0 = exp2_fast((m_run - Mu) * sl2);
    f1 = exp2_fast((m1 - Mu) * sl2);
    L = __builtin_fmaf(l1, f1, l_row * f0);
  }
  const float inv = L == 0.f ? 0.f : 1.f / L;
  const int i = p0 + row / p.g;
  const int hq = h * p.g + row % p.g;
  uint16_t* orow = p.out + (int64_t)(q_start + i) * p.out_stride + hq * kD + 4 * half;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // registers 4j..4j+3: d = 32dt + 8j + 4*half + 0..3
      float v4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * j + e;
        if constexpr (kParities == 2)
          v4[e] = __builtin_fmaf(mo[(rg * 64 + dt * 16 + r) * kWave + lane], f1, o[dt][r] * f0) * inv;
        else
          v4[e] = o[dt][r] * inv;
      }
      uint2 w;
      w.x = cvt_bf16x2(v4[0], v4[1]);
      w.y = cvt_bf16x2(v4[2], v4[3]);
      *(uint2*)(orow + 32 * dt + 8 * j) = w;
    }
  }
}

}  // namespace prefill
}  // namespace sd
