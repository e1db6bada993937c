// Tile loads shared by the decode kernels that take one 64-token tile per
// wave (decode_fold.hip, decode_cb.hip): buffer resources of one (batch,
// kv-head), the metadata words of a tile, and the lane-pair swap.
#pragma once
#include "decode_common.hpp"

namespace mz {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// Buffer resources of one (batch, kv-head): the packed prefix and metadata
// (bounded by their filled length, so a load past it reads 0, never faults).
struct Bufs {
  __amdgpu_buffer_rsrc_t kp, vp, kmn, ksc, vmn, vsc;
  // first residual row of this (batch, kv-head); each residual tile bounds its
  // own buffer by its filled rows (padding tokens read 0)
  const uint16_t* kr;
  const uint16_t* vr;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_buf(const void* p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)bytes, 0x00020000);
}

// Metadata words of a tile: MW = 1 (fp16 / bf16: one word holds both entries) or 2 (fp32).
template <int MW>
struct MetaWords {
  uint32_t kmn[MW], ksc[MW];  // key groups of channels 2*lane, 2*lane+1 (raw bits)
  uint32_t vmn[MW], vsc[MW];  // value groups 0, 1 of token lane (raw bits)
};

template <int MW>
__device__ __forceinline__ float2 meta_cvt(const uint32_t (&w)[MW], int dt) {
  if constexpr (MW == 2) {
    return float2{__builtin_bit_cast(float, w[0]), __builtin_bit_cast(float, w[1])};
  } else {
    if (dt == MZ_F16) return float2{h2f((uint16_t)w[0]), h2f((uint16_t)(w[0] >> 16))};
    return float2{bf2f((uint16_t)w[0]), bf2f((uint16_t)(w[0] >> 16))};
  }
}

template <int MW>
__device__ __forceinline__ void load_meta(uint32_t (&w)[MW], const __amdgpu_buffer_rsrc_t& r, int voff, int soff) {
  w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
  if constexpr (MW == 2) w[1] = __builtin_amdgcn_raw_buffer_load_b32(r, voff + 4, soff, 0);
}

// All metadata of a tile (loaded one tile ahead of its use).  HD = head_dim
// (64 or 128): HD / 64 value groups per token; with HD = 64 the key entries
// of lanes 32..63 lie past the tile's own (they are not used).
template <int MW, int HD>
__device__ __forceinline__ void load_meta_tile(MetaWords<MW>& t, const Bufs& bf, int tile, int lane) {
  constexpr int ES = 2 * MW;  // bytes per metadata entry
  constexpr int NGH = HD / 64;
  const int kmo = 2 * lane * ES, kms = tile * HD * ES;
  load_meta<MW>(t.kmn, bf.kmn, kmo, kms);
  load_meta<MW>(t.ksc, bf.ksc, kmo, kms);
  const int vmo = NGH * lane * ES, vms = tile * 64 * NGH * ES;
  if constexpr (NGH == 1 && MW == 1) {
    // one 16-bit entry per token: a 32-bit read would reach past the buffer's
    // end at the last token of the last tile (and then read 0 as a whole)
    t.vmn[0] = __builtin_amdgcn_raw_buffer_load_b16(bf.vmn, vmo, vms, 0);
    t.vsc[0] = __builtin_amdgcn_raw_buffer_load_b16(bf.vsc, vmo, vms, 0);
  } else {
    load_meta<MW>(t.vmn, bf.vmn, vmo, vms);
    load_meta<MW>(t.vsc, bf.vsc, vmo, vms);
  }
}

// Logit v (base-2 units) plus the additive mask entry m, times log2(e).
// Finite entries below -2^127 (the finfo.min masks of the 16-bit and fp32
// dtypes) are raised to -2^127 first so the product stays finite: a row that
// such entries mask everywhere then has equal logits and averages its values,
// as the reference's softmax does over its equal shifted logits; -inf (the
// boolean mask's excluded tokens) and NaN pass unchanged.
__device__ __forceinline__ float add_mask_log2(float v, float m) {
  const float mc = (m > -INFINITY && m < -0x1p127f) ? -0x1p127f : m;
  return __builtin_fmaf(mc, 1.44269504088896341f, v);
}

// The word of the other lane of this lane's pair (lanes 2m, 2m+1).
__device__ __forceinline__ uint32_t dpp_swap_pairs(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, DPP_QUAD_XOR1, 0xF, 0xF, true);
}

}  // namespace mz
