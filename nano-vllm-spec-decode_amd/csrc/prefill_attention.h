// Internal interface between the varlen entry point and the prefill kernel (prefill_attention.hip).
#pragma once
#include "sd_common.h"

namespace sd {

// Sequences with at most this many queries in a varlen call take the residue kernel (the decode / verify
// arithmetic, bitwise equal to sd_paged_decode); longer query runs take the prefill kernel.
constexpr int kResidueMaxQ = 16;
// Rows (query position x query head of one KV head) per prefill workgroup.
constexpr int kPrefillRows = 128;

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_stride;             // elements between consecutive query tokens (head stride 128)
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_stride, v_stride;   // elements between consecutive key tokens / cache slots
  const int32_t* block_tables;  // null: keys are rows cu_k[s] + j of k / v
  int32_t table_width;
  int32_t block_size;
  int64_t num_blocks;
  const int32_t* cu_q;
  const int32_t* cu_k;
  const int32_t* work;          // (sequence, q-block) pairs written by varlen_plan
  const int32_t* work_count;
  int32_t max_items;            // grid size (upper bound of *work_count)
  int32_t total_q;
  int64_t total_k;
  int32_t Hkv, g, P;            // P = query positions per q-block (P * g <= kPrefillRows)
  float scale_log2;             // softmax scale * log2(e)
  uint16_t* out;
  int64_t out_stride;
};

// Enqueues the prefill kernel; returns a Status.
int launch_prefill(const PrefillArgs& a, hipStream_t stream);

}  // namespace sd
