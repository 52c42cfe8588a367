// Paged attention for decode / speculative verify (replaces flash_attn_with_kvcache,
// nanovllm/layers/attention.py:71-78) and for varlen prefill / mixed prefill+decode (replaces
// flash_attn_varlen_func, attention.py:64-70). One kernel family serves both.
//
// Work decomposition. A work item is (sequence, query group, KV head, key split):
//   * query group: P consecutive query positions of one sequence; with g = Hq/Hkv heads sharing the KV
//     head, the group holds P*g "rows" (row r = position r/g, head r%g) — GQA head-group sharing: the
//     KV stream is read once for all g query heads.
//   * key split: a fixed 512-token range [512*s, 512*(s+1)) of the keys. Split boundaries never depend on
//     batch size, query count or context length, and partial results are merged in a fixed order, so a
//     row's output is bitwise independent of the batch it runs in (decode vs verify vs mixed).
// A 256-thread workgroup (4 waves) handles one item. Each wave streams 32-key tiles j = first + wave,
// first + wave + 4, ... : 16-byte coalesced global loads into registers (the next tile is in flight
// while the current one is computed), a wave-private LDS stage (rows padded to 272 B so both the K
// reads and the transposed V reads below are bank-conflict free), then bf16 MFMA 32x32x16:
//   S^T[32 keys x 32 rows] = K[32 x 128] . Q^T         (A = K from LDS, B = Q in registers)
//   O^T[128 d x 32 rows]  += V^T[128 x 32] . P^T        (A = V^T gathered from LDS, B = P in registers)
// S^T's accumulator layout gives each lane one row and 16 keys, so the online softmax needs one
// cross-lane exchange (lane ^ 32) per reduction, and P feeds the second MFMA straight from registers
// (the key order inside each 16-key k-step is permuted identically for P and V^T). The four waves'
// (max, sum, O) are merged in LDS in wave order; a split that is the sequence's only one writes bf16
// output directly, otherwise fp32 partials go to the workspace and attn_combine merges splits in order.
#include <math.h>

#include "sd_common.h"
#include "../../include/sd_attn.h"

namespace sd {
namespace {

constexpr int kD = 128;                        // head_dim (Qwen3)
constexpr int kTile = 32;                      // keys per wave step
constexpr int kWaves = 4;                      // waves per workgroup
constexpr int kSplit = 512;                    // keys per split
constexpr int kLdsRow = 272;                   // bytes per staged key row: 256 + 16 pad
constexpr int kLdsTensor = kTile * kLdsRow;    // one 32-key tile of K (or V)
constexpr int kLdsWave = 2 * kLdsTensor;       // K tile then V tile
constexpr int kLdsBytes = kWaves * kLdsWave;   // 69,632 B: two workgroups fit a CU's 160 KB
constexpr int kObRow = kD + 4;                 // fp32 row stride of the cross-wave O buffer (bank padding)

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
  const int32_t* cu_q;          // varlen
  const int32_t* cu_k;          // varlen
  const int32_t* work;          // varlen: (sequence, group) pairs
  const int32_t* work_count;    // varlen: number of valid pairs
  int32_t n;                    // decode: queries per sequence
  int32_t groups_per_seq;       // decode: ceil(n / P)
  int32_t total_q;              // tokens in q
  int64_t total_k;              // varlen without block table: rows in k / v
  int32_t Hq, Hkv, g, P;
  int32_t nsplit;               // grid.x: splits allocated per item
  int32_t rows_alloc;           // rows per (item, head, split) partial
  float scale_log2;             // softmax scale * log2(e)
  uint16_t* out;
  int64_t out_stride;
  float* part_o;                // [item][Hkv][nsplit][rows_alloc][kD]
  float* part_ml;               // [item][Hkv][nsplit][rows_alloc][2] = (max, sum)
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
    it.seq = item / p.groups_per_seq;
    grp = item % p.groups_per_seq;
    it.q_start = it.seq * p.n;
    it.Lq = p.n;
    it.Lk = p.context_lens[it.seq];
    if (it.Lk < 0) it.Lk = 0;
  }
  if (p.block_tables && (int64_t)it.Lk > (int64_t)p.table_width * p.block_size)
    it.Lk = p.table_width * p.block_size;  // never index past the table row
  if ((int64_t)it.Lk > (int64_t)p.nsplit * kSplit) it.Lk = p.nsplit * kSplit;  // never past the allocated splits
  it.p0 = grp * p.P;
  it.np = min(p.P, it.Lq - it.p0);
  if (it.np <= 0) return it;
  it.kmax = min(max(it.Lk - it.Lq + it.p0 + it.np, 0), it.Lk);
  it.valid = true;
  return it;
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

template <int MT, bool kVarlen, bool kPaged>
__global__ __launch_bounds__(kWaves * kWave) void attn_fwd(Params p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];

  const int split = blockIdx.x;
  const int h = blockIdx.y;
  const int item = blockIdx.z;
  const Item it = describe<kVarlen>(p, item);
  if (!it.valid) return;
  const int nsplit_act = (it.kmax + kSplit - 1) / kSplit;
  const int rows = it.np * p.g;
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int r = lane % 32;   // row (within a 32-row tile) owned by this lane
  const int hh = lane / 32;  // which half of the k / key sub-blocks this lane holds

  if (it.kmax <= 0) {  // no row sees any key (e.g. context_len 0 padding): zeros, written once
    if (split != 0) return;
    for (int e = tid; e < rows * (kD / 8); e += kWaves * kWave) {
      const int row = e / (kD / 8), c = e % (kD / 8);
      const int i = it.p0 + row / p.g, hq = h * p.g + row % p.g;
      *(u32x4*)(p.out + (int64_t)(it.q_start + i) * p.out_stride + hq * kD + c * 8) = u32x4{0, 0, 0, 0};
    }
    return;
  }
  if (split >= nsplit_act) return;
  const int kbeg = split * kSplit;
  const int kend = min(kbeg + kSplit, it.kmax);

  // Per-row visible-key limit inside this split (bottom-right causal: query i sees Lk - Lq + i + 1 keys).
  int lim[MT];
  bf16x8 qv[MT][8];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int row = mt * 32 + r;
    if (row < rows) {
      const int i = it.p0 + row / p.g;
      const int hq = h * p.g + row % p.g;
      lim[mt] = min(max(it.Lk - it.Lq + i + 1, 0), kend);
      const uint16_t* qp = p.q + (int64_t)(it.q_start + i) * p.q_stride + hq * kD + 64 * hh;
#pragma unroll
      for (int s = 0; s < 8; ++s) qv[mt][s] = *(const bf16x8*)(qp + 8 * s);
    } else {
      lim[mt] = kend;  // padding row: Q = 0 keeps its scores finite; never written
#pragma unroll
      for (int s = 0; s < 8; ++s) qv[mt][s] = bf16x8{};
    }
  }

  float m[MT], l[MT];
  f32x16 o[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    m[mt] = -INFINITY;
    l[mt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[mt][dt] = f32x16{};
  }

  uint8_t* kl = lds + wave * kLdsWave;
  uint8_t* vl = kl + kLdsTensor;
  // Staging layout: load q covers keys 4q .. 4q+3, 16 lanes per key row, 16 B per lane.
  const int st_key = lane / 16;
  const int st_chunk = lane % 16;
  u32x4 sk[8], sv[8];

  auto load_tile = [&](int jt) {
    const int t0 = jt * kTile;
    const uint16_t* kb = nullptr;
    const uint16_t* vb = nullptr;
    int nvalid = min(kTile, kend - t0);
    if (kPaged) {
      const int bi = t0 / p.block_size;
      const int blk = bi < p.table_width ? p.block_tables[(int64_t)it.seq * p.table_width + bi] : -1;
      if (blk < 0 || blk >= p.num_blocks) {
        nvalid = 0;  // invalid block id reads as zeros instead of faulting
      } else {
        const int64_t slot0 = (int64_t)blk * p.block_size + t0 % p.block_size;
        kb = p.k + slot0 * p.k_stride + h * kD;
        vb = p.v + slot0 * p.v_stride + h * kD;
      }
    } else {
      const int64_t row0 = (int64_t)p.cu_k[it.seq] + t0;
      kb = p.k + row0 * p.k_stride + h * kD;
      vb = p.v + row0 * p.v_stride + h * kD;
    }
#pragma unroll
    for (int qd = 0; qd < 8; ++qd) {
      const int tt = 4 * qd + st_key;
      if (tt < nvalid) {
        sk[qd] = *(const u32x4*)(kb + (int64_t)tt * p.k_stride + st_chunk * 8);
        sv[qd] = *(const u32x4*)(vb + (int64_t)tt * p.v_stride + st_chunk * 8);
      } else {
        sk[qd] = u32x4{0, 0, 0, 0};
        sv[qd] = u32x4{0, 0, 0, 0};
      }
    }
  };

  auto store_tile = [&]() {
#pragma unroll
    for (int qd = 0; qd < 8; ++qd) {
      const int off = (4 * qd + st_key) * kLdsRow + st_chunk * 16;
      *(u32x4*)(kl + off) = sk[qd];
      *(u32x4*)(vl + off) = sv[qd];
    }
  };

  // K operand (A of S^T): lane holds key r, d = 64*hh + 8*ks + e for k-step ks.
  const uint8_t* k_rd = kl + r * kLdsRow + hh * 128;
  // V^T operand (A of O^T): lane holds d = 32*dt + r, keys 16*s2 + 4*hh + (e%4) + 8*(e/4).
  const uint8_t* v_rd = vl + (4 * hh) * kLdsRow + r * 2;

  auto compute_tile = [&](int jt) {
    const int t0 = jt * kTile;
    f32x16 s[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) s[mt] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const bf16x8 a = *(const bf16x8*)(k_rd + ks * 16);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) s[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qv[mt][ks], s[mt], 0, 0, 0);
    }

    bf16x8 pb[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      float x[16];
      float mx = -INFINITY;
#pragma unroll
      for (int idx = 0; idx < 16; ++idx) {
        const int tok = t0 + 8 * (idx / 4) + 4 * hh + (idx % 4);
        x[idx] = tok < lim[mt] ? s[mt][idx] * p.scale_log2 : -INFINITY;
        mx = fmaxf(mx, x[idx]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m[mt], mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = exp2_fast(m[mt] - m_use);
      float sum = 0.f;
#pragma unroll
      for (int idx = 0; idx < 16; ++idx) {
        x[idx] = exp2_fast(x[idx] - m_use);
        sum += x[idx];
      }
      sum += __shfl_xor(sum, 32);
      l[mt] = l[mt] * alpha + sum;
      m[mt] = m_new;
      if (!__all(alpha == 1.f)) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[mt][dt] *= alpha;
      }
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        u32x4 w;
        w[0] = pack_bf16x2(x[8 * s2 + 0], x[8 * s2 + 1]);
        w[1] = pack_bf16x2(x[8 * s2 + 2], x[8 * s2 + 3]);
        w[2] = pack_bf16x2(x[8 * s2 + 4], x[8 * s2 + 5]);
        w[3] = pack_bf16x2(x[8 * s2 + 6], x[8 * s2 + 7]);
        pb[mt][s2] = __builtin_bit_cast(bf16x8, w);
      }
    }

#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        uint16_t e16[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          e16[e] = *(const uint16_t*)(v_rd + (16 * s2 + (e % 4) + 8 * (e / 4)) * kLdsRow + dt * 64);
        u32x4 w;
        w[0] = (uint32_t)e16[0] | ((uint32_t)e16[1] << 16);
        w[1] = (uint32_t)e16[2] | ((uint32_t)e16[3] << 16);
        w[2] = (uint32_t)e16[4] | ((uint32_t)e16[5] << 16);
        w[3] = (uint32_t)e16[6] | ((uint32_t)e16[7] << 16);
        const bf16x8 va = __builtin_bit_cast(bf16x8, w);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          o[mt][dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb[mt][s2], o[mt][dt], 0, 0, 0);
      }
    }
  };

  const int first_tile = kbeg / kTile;
  const int end_tile = (kend + kTile - 1) / kTile;
  int j = first_tile + wave;
  if (j < end_tile) load_tile(j);
  while (j < end_tile) {
    lds_wave_fence();  // this wave's reads of the previous tile are done before it is overwritten
    store_tile();
    lds_wave_fence();  // the tile is in LDS before any lane reads it
    const int jn = j + kWaves;
    if (jn < end_tile) load_tile(jn);  // next tile's global loads overlap this tile's math
    compute_tile(j);
    j = jn;
  }

  // ---- merge the four waves in wave order ----
  __syncthreads();
  float* ml = (float*)lds;                    // [wave][MT*32 rows][2]
  float* ob = (float*)(lds + 4096);           // [MT*32 rows][kObRow]
  if (hh == 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      ml[(wave * MT * 32 + mt * 32 + r) * 2 + 0] = m[mt];
      ml[(wave * MT * 32 + mt * 32 + r) * 2 + 1] = l[mt];
    }
  }
  __syncthreads();
  float Mrow[MT], Lrow[MT], fself[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int row = mt * 32 + r;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, ml[(w * MT * 32 + row) * 2]);
    const float M_use = M == -INFINITY ? 0.f : M;
    float L = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) L += ml[(w * MT * 32 + row) * 2 + 1] * exp2_fast(ml[(w * MT * 32 + row) * 2] - M_use);
    Mrow[mt] = M;
    Lrow[mt] = L;
    fself[mt] = exp2_fast(m[mt] - M_use);
  }
  for (int w = 0; w < kWaves; ++w) {
    if (wave == w) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        float* orow = ob + (mt * 32 + r) * kObRow;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            f32x4 val;
#pragma unroll
            for (int i = 0; i < 4; ++i) val[i] = o[mt][dt][4 * jj + i] * fself[mt];
            const int d = 32 * dt + 8 * jj + 4 * hh;
            if (w > 0) val = *(const f32x4*)(orow + d) + val;
            if (w < kWaves - 1) {
              *(f32x4*)(orow + d) = val;
            } else {
#pragma unroll
              for (int i = 0; i < 4; ++i) o[mt][dt][4 * jj + i] = val[i];
            }
          }
        }
      }
    }
    if (w < kWaves - 1) __syncthreads();
  }
  if (wave != kWaves - 1) return;

  // ---- write: bf16 output (only split) or fp32 partial ----
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int row = mt * 32 + r;
    if (row >= rows) continue;
    const int i = it.p0 + row / p.g;
    const int hq = h * p.g + row % p.g;
    if (nsplit_act == 1) {
      const float L = Lrow[mt];
      uint16_t* op = p.out + (int64_t)(it.q_start + i) * p.out_stride + hq * kD;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          float v4[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v4[e] = L == 0.f ? 0.f : o[mt][dt][4 * jj + e] / L;
          uint2 w2;
          w2.x = pack_bf16x2(v4[0], v4[1]);
          w2.y = pack_bf16x2(v4[2], v4[3]);
          *(uint2*)(op + 32 * dt + 8 * jj + 4 * hh) = w2;
        }
      }
    } else {
      const int64_t base = (((int64_t)item * p.Hkv + h) * p.nsplit + split) * p.rows_alloc + row;
      float* po = p.part_o + base * kD;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          f32x4 val;
#pragma unroll
          for (int e = 0; e < 4; ++e) val[e] = o[mt][dt][4 * jj + e];
          *(f32x4*)(po + 32 * dt + 8 * jj + 4 * hh) = val;
        }
      }
      if (hh == 0) {
        p.part_ml[base * 2 + 0] = Mrow[mt];
        p.part_ml[base * 2 + 1] = Lrow[mt];
      }
    }
  }
}

// Merges the fp32 split partials of items with more than one active split, in split order.
template <bool kVarlen>
__global__ __launch_bounds__(256) void attn_combine(Params p) {
  const int item = blockIdx.x;
  const int h = blockIdx.y;
  const Item it = describe<kVarlen>(p, item);
  if (!it.valid) return;
  const int nsplit_act = (it.kmax + kSplit - 1) / kSplit;
  if (nsplit_act <= 1) return;
  const int rows = it.np * p.g;
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  for (int row = wave; row < rows; row += 4) {
    const int64_t base0 = (((int64_t)item * p.Hkv + h) * p.nsplit) * p.rows_alloc + row;
    float M = -INFINITY;
    for (int s = 0; s < nsplit_act; ++s) M = fmaxf(M, p.part_ml[(base0 + (int64_t)s * p.rows_alloc) * 2]);
    const float M_use = M == -INFINITY ? 0.f : M;
    float L = 0.f, o0 = 0.f, o1 = 0.f;
    for (int s = 0; s < nsplit_act; ++s) {
      const int64_t b = base0 + (int64_t)s * p.rows_alloc;
      const float f = exp2_fast(p.part_ml[b * 2] - M_use);
      L += p.part_ml[b * 2 + 1] * f;
      const float2 ov = *(const float2*)(p.part_o + b * kD + 2 * lane);
      o0 += ov.x * f;
      o1 += ov.y * f;
    }
    const int i = it.p0 + row / p.g;
    const int hq = h * p.g + row % p.g;
    uint16_t* op = p.out + (int64_t)(it.q_start + i) * p.out_stride + hq * kD;
    const float r0 = L == 0.f ? 0.f : o0 / L;
    const float r1 = L == 0.f ? 0.f : o1 / L;
    *(uint32_t*)(op + 2 * lane) = pack_bf16x2(r0, r1);
  }
}

// Varlen work list: every sequence contributes ceil(Lq / P) (sequence, group) items, in order.
__global__ __launch_bounds__(256) void varlen_plan(const int32_t* __restrict__ cu_q, int32_t num_seqs, int32_t P,
                                                   int32_t* __restrict__ work, int32_t* __restrict__ count,
                                                   int32_t max_items) {
  __shared__ int32_t scan[256];
  __shared__ int32_t carry;
  const int tid = threadIdx.x;
  if (tid == 0) carry = 0;
  __syncthreads();
  for (int base = 0; base < num_seqs; base += 256) {
    const int s = base + tid;
    int ng = 0;
    if (s < num_seqs) {
      const int Lq = cu_q[s + 1] - cu_q[s];
      ng = Lq > 0 ? (Lq + P - 1) / P : 0;
    }
    scan[tid] = ng;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
      const int add = tid >= off ? scan[tid - off] : 0;
      __syncthreads();
      scan[tid] += add;
      __syncthreads();
    }
    const int start = carry + scan[tid] - ng;
    for (int gi = 0; gi < ng; ++gi) {
      if (start + gi < max_items) {
        work[2 * (start + gi)] = s;
        work[2 * (start + gi) + 1] = gi;
      }
    }
    __syncthreads();
    if (tid == 255) carry += scan[255];
    __syncthreads();
  }
  if (tid == 0) *count = min(carry, max_items);
}

constexpr float kLog2e = 1.4426950408889634f;

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct Layout {
  size_t part_o, part_ml, work, count, total;
};

Layout workspace_layout(int64_t items, int Hkv, int nsplit, int rows_alloc, bool varlen) {
  Layout L;
  const int64_t cells = items * Hkv * nsplit * rows_alloc;
  L.part_o = 0;
  L.part_ml = align256(L.part_o + (size_t)cells * kD * sizeof(float));
  L.work = align256(L.part_ml + (size_t)cells * 2 * sizeof(float));
  L.count = align256(L.work + (varlen ? (size_t)items * 2 * sizeof(int32_t) : 0));
  L.total = align256(L.count + (varlen ? sizeof(int32_t) : 0));
  return L;
}

// Row tiles per workgroup and positions per query group for g query heads per KV head.
void decode_shape(int n, int g, int* MT, int* P) {
  if (n * g <= 32) {
    *MT = 1;
    *P = n;
  } else {
    *MT = 2;
    *P = min(n, 64 / g);
  }
}

int check_heads(const char* who, int Hq, int Hkv, int D) {
  if (D != kD) return fail(kUnsupported, "%s: head_dim %d not supported (only %d)", who, D, kD);
  if (Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0)
    return fail(kBadArgument, "%s: num_heads %d must be a positive multiple of num_kv_heads %d", who, Hq, Hkv);
  if (Hq / Hkv > 64) return fail(kUnsupported, "%s: more than 64 query heads per KV head", who);
  return kOk;
}

}  // namespace
}  // namespace sd

using namespace sd;

extern "C" size_t sd_paged_decode_workspace_size(int32_t num_seqs, int32_t num_query_tokens, int32_t num_heads,
                                                 int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                                 int32_t table_width) {
  if (num_seqs <= 0 || num_query_tokens <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads) return 0;
  (void)head_dim;
  int MT, P;
  decode_shape(num_query_tokens, num_heads / num_kv_heads, &MT, &P);
  const int groups = (num_query_tokens + P - 1) / P;
  const int nsplit = (int)(((int64_t)table_width * block_size + kSplit - 1) / kSplit);
  return workspace_layout((int64_t)num_seqs * groups, num_kv_heads, max(nsplit, 1), MT * 32, false).total;
}

extern "C" int sd_paged_decode(const void* q, int64_t q_token_stride, const void* k_cache, const void* v_cache,
                               int64_t num_blocks, int32_t block_size, const int32_t* context_lens,
                               const int32_t* block_tables, int32_t table_width, int32_t num_seqs,
                               int32_t num_query_tokens, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                               float scale, void* out, int64_t out_token_stride, void* workspace,
                               size_t workspace_bytes, void* stream) {
  const char* who = "sd_paged_decode";
  int rc = check_heads(who, num_heads, num_kv_heads, head_dim);
  if (rc) return rc;
  if (num_seqs < 0 || num_query_tokens <= 0 || table_width <= 0 || num_blocks <= 0)
    return fail(kBadArgument, "%s: bad sizes (seqs %d, queries %d, table width %d, blocks %lld)", who, num_seqs,
                num_query_tokens, table_width, (long long)num_blocks);
  if (block_size <= 0 || block_size % kTile)
    return fail(kUnsupported, "%s: block_size %d must be a positive multiple of %d", who, block_size, kTile);
  if (num_seqs == 0) return kOk;
  if (!q || !k_cache || !v_cache || !context_lens || !block_tables || !out)
    return fail(kBadArgument, "%s: null pointer", who);
  if (q_token_stride < (int64_t)num_heads * head_dim || out_token_stride < (int64_t)num_heads * head_dim)
    return fail(kBadArgument, "%s: token stride smaller than num_heads*head_dim", who);
  if (((uintptr_t)q | (uintptr_t)out | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16 || q_token_stride % 8 ||
      out_token_stride % 8)
    return fail(kUnsupported, "%s: q / out / caches must be 16-byte aligned with strides multiple of 8", who);
  const int g = num_heads / num_kv_heads;
  int MT, P;
  decode_shape(num_query_tokens, g, &MT, &P);
  const int groups = (num_query_tokens + P - 1) / P;
  const int64_t items = (int64_t)num_seqs * groups;
  const int nsplit = max(1, (int)(((int64_t)table_width * block_size + kSplit - 1) / kSplit));
  if (items > 65535) return fail(kUnsupported, "%s: %lld work items exceed the grid limit", who, (long long)items);
  const Layout lay = workspace_layout(items, num_kv_heads, nsplit, MT * 32, false);
  if (!workspace || workspace_bytes < lay.total)
    return fail(kWorkspaceTooSmall, "%s: workspace %zu B < %zu B", who, workspace_bytes, lay.total);

  Params p{};
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
  p.nsplit = nsplit;
  p.rows_alloc = MT * 32;
  p.scale_log2 = scale * kLog2e;
  p.out = (uint16_t*)out;
  p.out_stride = out_token_stride;
  p.part_o = (float*)((uint8_t*)workspace + lay.part_o);
  p.part_ml = (float*)((uint8_t*)workspace + lay.part_ml);

  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(nsplit, num_kv_heads, (unsigned)items), block(kWaves * kWave);
  if (MT == 1)
    hipLaunchKernelGGL((attn_fwd<1, false, true>), grid, block, 0, s, p);
  else
    hipLaunchKernelGGL((attn_fwd<2, false, true>), grid, block, 0, s, p);
  if ((rc = check_launch(who))) return rc;
  if (nsplit > 1) {
    hipLaunchKernelGGL((attn_combine<false>), dim3((unsigned)items, num_kv_heads), dim3(256), 0, s, p);
    if ((rc = check_launch(who))) return rc;
  }
  return kOk;
}

namespace {
int64_t varlen_items(int32_t num_seqs, int32_t total_q, int P) { return (int64_t)(total_q + P - 1) / P + num_seqs; }
}  // namespace

extern "C" size_t sd_varlen_workspace_size(int32_t num_seqs, int32_t total_q, int32_t max_seqlen_k, int32_t num_heads,
                                           int32_t num_kv_heads, int32_t head_dim) {
  if (num_seqs <= 0 || total_q <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads) return 0;
  (void)head_dim;
  const int P = max(1, 64 / (num_heads / num_kv_heads));
  const int nsplit = max(1, (max_seqlen_k + kSplit - 1) / kSplit);
  return workspace_layout(varlen_items(num_seqs, total_q, P), num_kv_heads, nsplit, 64, true).total;
}

extern "C" int sd_varlen_attention(const void* q, int64_t q_token_stride, const void* k, int64_t k_token_stride,
                                   const void* v, int64_t v_token_stride, int64_t total_k, int64_t num_blocks,
                                   int32_t block_size, const int32_t* block_tables, int32_t table_width,
                                   const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int32_t num_seqs,
                                   int32_t total_q, int32_t max_seqlen_q, int32_t max_seqlen_k, int32_t num_heads,
                                   int32_t num_kv_heads, int32_t head_dim, float scale, void* out,
                                   int64_t out_token_stride, void* workspace, size_t workspace_bytes, void* stream) {
  const char* who = "sd_varlen_attention";
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
  } else if (k_token_stride < (int64_t)num_kv_heads * head_dim || v_token_stride < (int64_t)num_kv_heads * head_dim) {
    return fail(kBadArgument, "%s: k / v token stride smaller than num_kv_heads*head_dim", who);
  }
  if (q_token_stride < (int64_t)num_heads * head_dim || out_token_stride < (int64_t)num_heads * head_dim)
    return fail(kBadArgument, "%s: token stride smaller than num_heads*head_dim", who);
  if (((uintptr_t)q | (uintptr_t)out | (uintptr_t)k | (uintptr_t)v) % 16 || q_token_stride % 8 ||
      out_token_stride % 8 || k_token_stride % 8 || v_token_stride % 8)
    return fail(kUnsupported, "%s: q / out / k / v must be 16-byte aligned with strides multiple of 8", who);
  const int g = num_heads / num_kv_heads;
  const int P = max(1, 64 / g);
  const int64_t items = varlen_items(num_seqs, total_q, P);
  if (items > 65535) return fail(kUnsupported, "%s: %lld work items exceed the grid limit", who, (long long)items);
  const int nsplit = max(1, (max_seqlen_k + kSplit - 1) / kSplit);
  const Layout lay = workspace_layout(items, num_kv_heads, nsplit, 64, true);
  if (!workspace || workspace_bytes < lay.total)
    return fail(kWorkspaceTooSmall, "%s: workspace %zu B < %zu B", who, workspace_bytes, lay.total);

  Params p{};
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
  p.nsplit = nsplit;
  p.rows_alloc = 64;
  p.scale_log2 = scale * kLog2e;
  p.out = (uint16_t*)out;
  p.out_stride = out_token_stride;
  p.part_o = (float*)((uint8_t*)workspace + lay.part_o);
  p.part_ml = (float*)((uint8_t*)workspace + lay.part_ml);
  int32_t* work = (int32_t*)((uint8_t*)workspace + lay.work);
  int32_t* count = (int32_t*)((uint8_t*)workspace + lay.count);
  p.work = work;
  p.work_count = count;

  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(varlen_plan, dim3(1), dim3(256), 0, s, cu_seqlens_q, num_seqs, P, work, count, (int32_t)items);
  if ((rc = check_launch(who))) return rc;
  const dim3 grid(nsplit, num_kv_heads, (unsigned)items), block(kWaves * kWave);
  if (paged)
    hipLaunchKernelGGL((attn_fwd<2, true, true>), grid, block, 0, s, p);
  else
    hipLaunchKernelGGL((attn_fwd<2, true, false>), grid, block, 0, s, p);
  if ((rc = check_launch(who))) return rc;
  if (nsplit > 1) {
    hipLaunchKernelGGL((attn_combine<true>), dim3((unsigned)items, num_kv_heads), dim3(256), 0, s, p);
    if ((rc = check_launch(who))) return rc;
  }
  return kOk;
}
