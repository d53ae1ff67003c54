// monosum_wave.h — one wave's scans of monosum increment pairs (DPP), shared
// by the device sampler and the attention softmax. Include after monosum.h
// with RLH_MONO_QUAL = __device__ __forceinline__.
#pragma once

// DPP moves of a pair: lanes the masks leave out, and lanes whose source is
// outside the row, read 0 (bound_ctrl): the identity pair.
template <int CTRL, int ROWS, int BANKS>
__device__ __forceinline__ MonoFn dpp_fn(MonoFn f) {
  MonoFn g;
  g.a0 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)f.a0, CTRL, ROWS, BANKS, true);
  g.a1 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)f.a1, CTRL, ROWS, BANKS, true);
  return g;
}

// Inclusive scan of the lanes' functions in lane order (lane i: lanes 0..i),
// by the gfx9 DPP sequence: row_shr 1, 2, 4, 8 inside each row of 16 lanes,
// then row_bcast 15 and 31 carry the rows' totals forward.
__device__ __forceinline__ MonoFn wave_scan_fn(MonoFn f) {
  f = mono_then(dpp_fn<0x111, 0xf, 0xf>(f), f);  // row_shr:1
  f = mono_then(dpp_fn<0x112, 0xf, 0xf>(f), f);  // row_shr:2
  f = mono_then(dpp_fn<0x114, 0xf, 0xe>(f), f);  // row_shr:4, lanes 4..15 of each row
  f = mono_then(dpp_fn<0x118, 0xf, 0xc>(f), f);  // row_shr:8, lanes 8..15
  f = mono_then(dpp_fn<0x142, 0xa, 0xf>(f), f);  // row_bcast:15 into rows 1 and 3
  f = mono_then(dpp_fn<0x143, 0xc, 0xf>(f), f);  // row_bcast:31 into rows 2 and 3
  return f;
}

// The exclusive form from the inclusive one: lane i gets lane i - 1's value
// (wave_shr:1), lane 0 the identity.
__device__ __forceinline__ MonoFn wave_excl_fn(MonoFn incl) { return dpp_fn<0x138, 0xf, 0xf>(incl); }

__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, int lane) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, lane);
}
__device__ __forceinline__ float readlane_f32(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Composition of all 64 lanes' functions in lane order, in every lane.
__device__ __forceinline__ MonoFn wave_total_fn(MonoFn f) {
  const MonoFn incl = wave_scan_fn(f);
  return MonoFn{readlane_u32(incl.a0, 63), readlane_u32(incl.a1, 63)};
}

