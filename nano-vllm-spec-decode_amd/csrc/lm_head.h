// LM head over the verify rows with the verifier's argmax pass in its epilogue (replaces, for the rows the
// verifier reads, ParallelLMHead.forward, nanovllm/layers/embed_head.py:56-68, and the first read of the
// logits by verify_drafts, nanovllm/layers/sampler.py:66).
//
// logits[m, n] = bf16(sum_k hidden[rows[m], k] * weight[n, k]): the library GEMM's contract (fp32
// accumulation, one round to bf16), with the logits_indices gather folded into the loads of hidden.
// Shapes at Qwen3-8B: M = S (K+1) = 320 token rows, H = 4096, V = 151936 vocabulary rows: 398 GFLOP over the
// 1.24 GB weight, about 320 FLOP per byte, at the bf16 ridge of this GPU (2.5 PF / 8 TB/s).
//
// One 8-wave workgroup owns 256 vocabulary rows and up to 320 token rows and walks H in stages of 32:
//   * each stage's weight tile (256 x 32, 16 KB) and hidden tile (up to 320 x 32, 20 KB) are loaded straight
//     into a ring of four LDS stages (global_load_lds_dwordx4), three stages ahead of the MFMAs: at ~12.5 B per
//     clock per CU, the weight stream needs tens of KB in flight per CU to cover HBM latency. Both operands are
//     packed so that a stage tile is contiguous (rows of a tile are otherwise 2 H bytes apart, and such 64-byte
//     row pieces streamed the weight at 4.3 TB/s and the hidden rows at 6.3 TB/s from L2, measured alone). LDS
//     rows of 64 bytes, the 16-byte chunk c of row r at slot c ^ ((r >> 2) & 3): conflict-free operand reads;
//   * wave w takes vocabulary rows 64 (w % 4) .. +64 and token rows 32 MB (w / 4) .. +32 MB: 2 x MB
//     v_mfma_f32_32x32x16_bf16 tiles D[n][m] = sum_k W[n][k] H[m][k] (A = weight rows, B = hidden rows, both
//     ds_read_b128 from LDS), MB <= 5, accumulating in fp32;
//   * epilogue: a lane holds 16 vocabulary entries of one token row per tile (the other 16 in lane l ^ 32); it
//     rounds them to bf16, optionally stores them (the logits, for a sampling pass that reads them again), and
//     reduces the first argmax (torch.argmax order) over the workgroup's 256 entries: its own entries in
//     index order, the lane pair, then the four vocabulary waves through LDS. One (value, index) per token row
//     and workgroup goes out; lm_head_merge folds them into the verifier's span statistics.
#pragma once
#include "sd_common.h"

namespace sd {
namespace lmhead {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kWave;           // 512
constexpr int kN = 256;                            // vocabulary rows per workgroup
constexpr int kK = 32;                             // hidden columns per stage
constexpr int kRowBytes = kK * 2;                  // one LDS row: 64 B = 4 chunks of 16 B
constexpr int kMaxMB = 5;                          // token blocks of 32 per wave (2 waves: 320 rows)
constexpr int kMaxRows = 2 * kMaxMB * 32;          // 320 token rows per workgroup
constexpr int kWBytes = kN * kRowBytes;            // 16 KB
constexpr int kHBytes = kMaxRows * kRowBytes;      // 20 KB
constexpr int kStageBytes = kWBytes + kHBytes;     // 36 KB
constexpr int kRing = 4;                           // LDS stages: loads run 3 stages ahead of the MFMAs
constexpr int kLdsBytes = kRing * kStageBytes;     // 144 KB
constexpr int kCpolNT = 2;                         // cache policy of a load: non-temporal

struct TileBest {  // first argmax of one token row over one workgroup's vocabulary rows
  float val;
  int32_t idx;
};

// Packed operands (contiguous stage tiles, so that every stage load reads whole 1 KB blocks):
//   weight  wp[t][s][r][c] = weight[kN t + r][32 s + c]  (t < tiles, s < H / 32, r < kN, c < 32; rows past the
//           vocabulary are 0), made once per model by lm_head_pack_weight (sd_lm_head_pack_weight);
//   hidden  hp[s][m][c] = hidden[rows[m]][32 s + c]  (m < Mpad; rows past M are 0), made per call by
//           lm_head_pack_hidden, which also applies the logits_indices gather.
struct Args {
  const uint16_t* hp;       // packed hidden [H/32][Mpad][32]
  int32_t Mpad;             // gridDim.y * token rows per workgroup
  int32_t M;                // token rows
  const uint16_t* wp;       // packed weight [tiles][H/32][kN][32]
  int32_t V, H;
  uint16_t* logits;         // null, or [M, V] bf16 with row stride logits_stride
  int64_t logits_stride;
  int32_t logits_vec;       // rows 8-byte aligned: 4 entries per store
  TileBest* best;           // [M][tiles], or null (no argmax)
  int32_t tiles;            // vocabulary tiles of kN rows
  // Tiles full.. (the last, partial round of workgroups) are cut into `splits` ranges of H each, one
  // workgroup per range, so that the last round fills the GPU; such a workgroup writes its fp32 sums to
  // `part` ([row of workgroups][tile - full][split][8 waves][2][MB][16][64 lanes]) and lm_head_fixup adds the
  // ranges in order and runs the epilogue. splits = 1: every tile whole (full = tiles). full and splits are
  // functions of (V, H) only and every row of workgroups uses them, so a token row's logits do not depend on
  // how many rows the call has. The sequential form (lm_head_gemm<MB, true>) runs a split tile's ranges one
  // after another in one workgroup and adds them in the same order in registers: the same sums, no `part`.
  int32_t full;
  int32_t splits;
  float* part;
};

// One thread per 16 bytes of the packed weight.
__global__ __launch_bounds__(256) void lm_head_pack_weight(const uint16_t* __restrict__ w, int32_t V, int32_t H,
                                                           int32_t tiles, uint16_t* __restrict__ wp) {
  const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;   // 16-byte chunk of the output
  const int S = H / 32;
  if (o >= (int64_t)tiles * S * kN * 4) return;
  const int c8 = (int)(o % 4);
  const int r = (int)((o / 4) % kN);
  const int64_t ts = o / (4 * kN);
  const int s = (int)(ts % S);
  const int t = (int)(ts / S);
  const int n = kN * t + r;
  u32x4 v = {0, 0, 0, 0};
  if (n < V) v = *(const u32x4*)(w + (int64_t)n * H + 32 * s + 8 * c8);
  *(u32x4*)(wp + o * 8) = v;
}

// One thread per 16 bytes of the packed hidden rows (the logits_indices gather; an index outside the table
// reads nothing and packs a zero row, and lm_head_poison marks its sequence).
__global__ __launch_bounds__(256) void lm_head_pack_hidden(const uint16_t* __restrict__ hidden, int64_t stride,
                                                           int32_t hidden_rows, const int64_t* __restrict__ rows,
                                                           int32_t M, int32_t Mpad, int32_t H, uint16_t* __restrict__ hp) {
  const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int S = H / 32;
  if (o >= (int64_t)S * Mpad * 4) return;
  const int c8 = (int)(o % 4);
  const int m = (int)((o / 4) % Mpad);
  const int s = (int)(o / (4 * (int64_t)Mpad));
  u32x4 v = {0, 0, 0, 0};
  if (m < M) {
    const int64_t r = rows ? rows[m] : (int64_t)m;
    if (r >= 0 && r < hidden_rows) v = *(const u32x4*)(hidden + r * stride + 32 * s + 8 * c8);
  }
  *(u32x4*)(hp + o * 8) = v;
}

// LDS byte offset of 16-byte chunk c (0..3) of row r: rows of 64 B, the chunk swizzled by bits 2..3 of the row,
// so that 16 consecutive rows at one chunk (an operand read's 16-lane pass) cover all 64 banks.
__device__ __forceinline__ uint32_t slot(int row, int chunk) {
  return row * kRowBytes + ((chunk ^ ((row >> 2) & 3)) << 4);
}

template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

typedef __attribute__((address_space(3))) void lds_void;

// Epilogue, per 32-token-row block of a tile. A lane holds 16 vocabulary entries of one token row for each of
// its two 32-row vocabulary blocks (the other 16 in lane l ^ 32): it rounds them to bf16, stores them if the
// logits are asked for, and takes the first argmax (index order) of its entries and its lane pair's. Returns
// it in every lane; token row m of the call (no store, the argmax still taken, for m >= M).
__device__ __forceinline__ TileBest block_best(const Args& a, const f32x16 (&acc)[2], int n_wave, int m) {
  const int half = (threadIdx.x % kWave) / 32;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int nf = n_wave + 32 * nb + 8 * g + 4 * half;  // first of 4 consecutive entries
      float v[4];
      uint16_t bits[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        bits[e] = f32_to_bf16_bits(acc[nb][4 * g + e]);
        v[e] = bf16_bits_to_f32(bits[e]);
      }
      if (a.logits && m < a.M) {
        uint16_t* dst = a.logits + (int64_t)m * a.logits_stride + nf;
        if (nf + 3 < a.V && a.logits_vec) {
          *(uint2*)dst = make_uint2((uint32_t)bits[0] | ((uint32_t)bits[1] << 16),
                                    (uint32_t)bits[2] | ((uint32_t)bits[3] << 16));
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (nf + e < a.V) dst[e] = bits[e];
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (nf + e < a.V && bv == bv && !(v[e] <= bv)) {  // index order within the lane: strictly larger
          bv = v[e];
          bi = nf + e;
        }
    }
  }
  const float ov = __shfl_xor(bv, 32);
  const int oi = __shfl_xor(bi, 32);
  if (better(ov, oi, bv, bi)) {
    bv = ov;
    bi = oi;
  }
  return TileBest{bv, bi};
}

// The four vocabulary waves' candidates of `rows` token rows (red[row][wave], in LDS, after a barrier), reduced
// in wave order into best[m][tile] by threads 0.. of the workgroup.
__device__ __forceinline__ void reduce_best(const Args& a, const TileBest* red, int rows, int m0, int tile) {
  if (!a.best) return;  // a plain linear layer: the logits only
  for (int mr = threadIdx.x; mr < rows; mr += blockDim.x) {
    const int m = m0 + mr;
    if (m >= a.M) continue;
    TileBest b = red[mr * 4];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      const TileBest o = red[mr * 4 + w];
      if (better(o.val, o.idx, b.val, b.idx)) b = o;
    }
    a.best[(int64_t)m * a.tiles + tile] = b;
  }
}

template <int MB, bool kSeq = false>
__global__ __launch_bounds__(kThreads) void lm_head_gemm(Args a) {
  static_assert(MB >= 1 && MB <= kMaxMB, "token blocks per wave");
  static_assert(!kSeq || MB <= 2, "the sequential ranges keep a second accumulator set");
  constexpr int kRows = 2 * MB * 32;               // token rows of this workgroup
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int wn = wave % 4, wm = wave / 4;
  // This workgroup's tile and range of H stages (the whole of H, or one range of a split tile).
  const int S = a.H / kK;
  int tile = blockIdx.x, split = -1, s_begin = 0, nstages = S;
  if (!kSeq && (int)blockIdx.x >= a.full) {
    const int j = blockIdx.x - a.full;
    tile = a.full + j / a.splits;
    split = j % a.splits;
    s_begin = split * S / a.splits;
    nstages = (split + 1) * S / a.splits - s_begin;
  }
  const int m0 = blockIdx.y * kRows;

  // Stage loads straight into LDS (global_load_lds_dwordx4: lane l's 16 bytes land at the instruction's LDS
  // base + 16 l, i.e. row l / 4, physical chunk l % 4 of a 16-row group; so the lane fetches the logical chunk
  // that the swizzle puts there: each instruction reads one contiguous 1 KB block of a packed operand). Waves
  // 0-3 load the weight tile (4 groups of 16 rows each), waves 4-7 the hidden tile (MB groups each).
  const int lrow = lane / 4, lchunk = (lane % 4) ^ ((lane / 16) & 3);
  const uint32_t lane_off = lrow * 32 + 8 * lchunk;   // elements within a 16-row group
  const bool wloader = wave < 4;
  constexpr int kLoads = MB > 4 ? MB : 4;          // instructions per stage of the busiest loader
  const int nloads = wloader ? 4 : MB;
  uint32_t loff[kLoads], goff[kLoads];             // LDS offset; element offset within the stage tile
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    const int g = wloader ? 4 * wave + i : MB * (wave - 4) + min(i, MB - 1);
    goff[i] = 16 * g * 32 + lane_off;
    loff[i] = (wloader ? 0 : kWBytes) + 16 * g * kRowBytes;
  }
  // Every workgroup walks its stages in order from s_begin, so the workgroups of a round read the same hidden
  // stage at about the same time, and the weight, read once, streams with the non-temporal policy: both keep
  // the hidden rows in L2 (FETCH_SIZE 2.39 -> 1.28 GB per call against rotated starts and default loads, and
  // 455 -> 443 us).
  auto issue = [&](int st) {
    uint8_t* ring = lds + (st % kRing) * kStageBytes;
    const int ks = s_begin + st;
    const uint16_t* base = wloader ? a.wp + ((int64_t)tile * S + ks) * (kN * kK)
                                   : a.hp + ((int64_t)ks * a.Mpad + m0) * kK;
#pragma unroll
    for (int i = 0; i < kLoads; ++i)
      if (i < nloads) {
        if (wloader)
          __builtin_amdgcn_global_load_lds((const void*)(base + goff[i]), (lds_void*)(ring + loff[i]), 16, 0, kCpolNT);
        else
          __builtin_amdgcn_global_load_lds((const void*)(base + goff[i]), (lds_void*)(ring + loff[i]), 16, 0, 0);
      }
  };
  // Waits until this wave's loads of a stage have landed, given how many later stages it has issued.
  auto wait_stage = [&](int later) {
    if (wloader) {
      if (later >= 3) wait_vm<12>(); else if (later == 2) wait_vm<8>(); else if (later == 1) wait_vm<4>(); else wait_vm<0>();
    } else {
      if (later >= 3) wait_vm<3 * MB>(); else if (later == 2) wait_vm<2 * MB>(); else if (later == 1) wait_vm<MB>();
      else wait_vm<0>();
    }
  };

  f32x16 acc[2][MB];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = f32x16{};

  const int col = lane % 32, half = lane / 32;
  // Operand fragments of one 16-deep step (ks 0 or 1) of ring slot `buf`.
  auto read_frags = [&](int buf, int ks, bf16x8 (&af)[2], bf16x8 (&bfr)[MB]) {
    const uint8_t* wbuf = lds + buf * kStageBytes;
    const uint8_t* hbuf = wbuf + kWBytes;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) af[nb] = *(const bf16x8*)(wbuf + slot(64 * wn + 32 * nb + col, 2 * ks + half));
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) bfr[mb] = *(const bf16x8*)(hbuf + slot(MB * 32 * wm + 32 * mb + col, 2 * ks + half));
  };
  auto mfmas = [&](const bf16x8 (&af)[2], const bf16x8 (&bfr)[MB]) {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        acc[nb][mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[nb], bfr[mb], acc[nb][mb], 0, 0, 0);
  };
  // The hand-off between stages sits in the middle of a stage: once this wave's second-step fragments of
  // stage s are in registers, it waits for stage s+1's loads and the barrier (after which every wave is done
  // reading stage s, so its slot takes stage s+4), reads stage s+1's first-step fragments, and only then
  // runs stage s's second-step MFMAs: operand reads overlap MFMAs on both sides of the barrier.
  auto handoff = [&](int next) {  // `next` = the stage about to be read
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    wait_stage(min(nstages - 1 - next, 2));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (next + 3 < nstages) issue(next + 3);
  };
  // The sequential form: a split tile's range r covers stages r S / splits .. (r + 1) S / splits - 1 (the
  // physical split's ranges); each is summed from zero, and the ranges are added in order into `sum`, as
  // lm_head_fixup adds them.
  const int nranges = kSeq && tile >= a.full ? a.splits : 1;
  int range = 0, range_end = S / nranges;
  f32x16 sum[2][kSeq ? MB : 1];
  auto fold = [&]() {
    if constexpr (kSeq) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          sum[nb][mb] = range == 0 ? acc[nb][mb] : sum[nb][mb] + acc[nb][mb];
          acc[nb][mb] = f32x16{};
        }
    }
  };
  bf16x8 a0[2], b0[MB], a1[2], b1[MB];
  for (int st = 0; st < 3 && st < nstages; ++st) issue(st);
  handoff(0);
  read_frags(0, 0, a0, b0);
  // The last stage is peeled: a loop body without a branch between the hand-off's operand reads and the
  // second-step MFMAs lets those MFMAs wait only for their own (older) reads, not for the next stage's.
  for (int s = 0; s + 1 < nstages; ++s) {
    read_frags(s % kRing, 1, a1, b1);
    mfmas(a0, b0);
    handoff(s + 1);
    read_frags((s + 1) % kRing, 0, a0, b0);
    mfmas(a1, b1);
    if constexpr (kSeq) {
      if (s + 1 == range_end) {  // stage s ends range `range` (registers only: no memory operation)
        fold();
        ++range;
        range_end = (range + 1) * S / nranges;
      }
    }
  }
  read_frags((nstages - 1) % kRing, 1, a1, b1);
  mfmas(a0, b0);
  mfmas(a1, b1);
  if constexpr (kSeq) {
    if (nranges > 1) {  // the last range, added last
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = sum[nb][mb] + acc[nb][mb];
    }
  }

  if (split >= 0) {
    // ---- one range of a split tile: the fp32 sums out, lm_head_fixup finishes the tile ----
    const int64_t range = (int64_t)blockIdx.y * (a.tiles - a.full) * a.splits + (blockIdx.x - a.full);
    float* dst = a.part + (range * kWaves + wave) * (2 * MB * 16 * kWave) + lane;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) dst[((nb * MB + mb) * 16 + r) * kWave] = acc[nb][mb][r];
    return;
  }
  // ---- epilogue: per token row, the first argmax over the workgroup's 256 vocabulary rows ----
  __syncthreads();  // every wave's last stage read: the ring is free for the reduction
  TileBest* red = (TileBest*)lds;  // [kRows][4]
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int mr = MB * 32 * wm + 32 * mb + col;  // token row within the workgroup
    const f32x16 blk[2] = {acc[0][mb], acc[1][mb]};
    const TileBest b = block_best(a, blk, tile * kN + 64 * wn, m0 + mr);
    if (half == 0) red[mr * 4 + wn] = b;
  }
  __syncthreads();
  reduce_best(a, red, kRows, m0, tile);
}

// The tiles split along H: one 4-wave workgroup per (split tile, 32-token-row block, row of GEMM workgroups)
// adds the ranges' sums in range order and finishes the block as lm_head_gemm's epilogue does. Wave w takes
// the vocabulary rows of the GEMM's wave w of the block's token half: 64 w .. 64 w + 63.
template <int MB>
__global__ __launch_bounds__(256) void lm_head_fixup(Args a) {
  __shared__ TileBest red[32 * 4];
  const int lane = threadIdx.x % kWave;
  const int wn = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int wm = blockIdx.y / MB, mb = blockIdx.y % MB;
  const int tile = a.full + blockIdx.x;
  const int m0 = blockIdx.z * (2 * MB * 32);       // first token row of the GEMM's row of workgroups
  constexpr int kPerWave = 2 * MB * 16 * kWave;
  const int64_t range0 = ((int64_t)blockIdx.z * (a.tiles - a.full) + blockIdx.x) * a.splits;
  const float* src = a.part + (range0 * kWaves + 4 * wm + wn) * kPerWave + mb * 16 * kWave + lane;
  f32x16 acc[2];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[nb][r] = src[(nb * MB * 16 + r) * kWave];
  for (int sp = 1; sp < a.splits; ++sp) {
    const float* p = src + (int64_t)sp * kWaves * kPerWave;
    float t[2][16];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) t[nb][r] = p[(nb * MB * 16 + r) * kWave];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[nb][r] += t[nb][r];
  }
  const int col = lane % 32;
  const int mr = MB * 32 * wm + 32 * mb + col;
  const TileBest b = block_best(a, acc, tile * kN + 64 * wn, m0 + mr);
  if (lane < 32) red[col * 4 + wn] = b;
  __syncthreads();
  reduce_best(a, red, 32, m0 + MB * 32 * wm + 32 * mb, tile);
}

}  // namespace lmhead
}  // namespace sd
