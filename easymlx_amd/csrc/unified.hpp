// One launch for a mixed batch (the unified ragged step of
// lib/python/easymlx/operations/kernels/unified_attention.py:290-609, which the
// reference runs as one Metal dispatch over all rows): the first ndec workgroups
// run a decode body (4-bit 4x4x4, 16x16x32 or FP8) on the single-token rows, the
// others the prefill body on the rows of sequences with more than one query
// token.  Workgroups
// start in index order, so the decode workgroups (few: the host sizes them to
// the decode rows' share of the work) take one slot on some compute units from
// the start and stream their pages beside the prefill's matrix work on the
// same units.  The two bodies share the LDS arena and nothing else.
#pragma once

#include "decode_affine.hpp"
#include "decode_fp8.hpp"
#include "decode_q4.hpp"
#include "prefill_affine.hpp"

namespace emx {

template <int GS, int HG>
__global__ __launch_bounds__(256, 2) void unified_q4(PrefillArgs p, DecodeArgs d, int ndec) {
  if ((int)blockIdx.x < ndec)
    decode_q4_body<GS, HG>(d, blockIdx.x, ndec, d.plan, d.kv_lens, d.block_tables, d.S, d.max_blocks);
  else
    prefill_body<4, GS, HG>(p, (int)blockIdx.x - ndec);
}

// The same over an FP8 (E4M3) cache: the FP8 decode body, then the prefill body
// on its FP8 geometry.  d.num_waves = 4 * ndec.
template <int HG>
__global__ __launch_bounds__(256, 2) void unified_fp8(PrefillArgs p, DecodeArgs d, int ndec) {
  if ((int)blockIdx.x < ndec)
    decode_fp8_body<HG>(d, blockIdx.x, ndec);
  else
    prefill_body<4, 128, HG, true>(p, (int)blockIdx.x - ndec);
}

// The same with the 16x16x32 decode body (8-bit pages, group 32, GQA 8).
// d.num_waves = 4 * ndec.
template <int BITS, int GS, int HG>
__global__ __launch_bounds__(256, 2) void unified_affine(PrefillArgs p, DecodeArgs d, int ndec) {
  if ((int)blockIdx.x < ndec)
    decode_affine_body<BITS, GS, HG>(d, blockIdx.x, ndec);
  else
    prefill_body<BITS, GS, HG>(p, (int)blockIdx.x - ndec);
}

}  // namespace emx
