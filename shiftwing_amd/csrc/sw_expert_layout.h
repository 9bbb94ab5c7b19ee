// Where a layer's routed experts lie in HBM.
//
// Every matrix is cut into tile-groups: 16 rows x one 128-wide quant group,
// tg = row_tile * groups_per_row + group.  A tile-group's codes take
// 64 lanes x BPL bytes (BPL 16 for int4, 12 for int3; the lane layout is in
// sw_moe_kernels.h) and its 16 per-row scales 64 bytes (f32).  Codes and
// scales of a tile-group sit together in one record:
//   gate/up record (per gate/up tile-group): [gate codes | up codes |
//                                             gate scales | up scales]
//   down record (per down tile-group):       [codes | scales]
// An expert is its I/16 x ngh gate/up records followed by its H/16 x ngi down
// records; experts follow one another.  A wave that streams a row tile reads
// whole records: few, large, contiguous requests, with the scales of a group
// next to its codes (separate scale arrays cost the memory system far more
// than their 8% of the bytes).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

namespace sw {

// One tiled matrix of one expert: codes of tile-group tg at base + tg * rs,
// its 16 row scales at base + tg * rs + so.
struct TileMat {
  const unsigned char *base;
  unsigned rs, so;
};
__host__ __device__ inline const unsigned char *tm_codes(const TileMat &m, size_t tg) { return m.base + tg * m.rs; }
__host__ __device__ inline const float *tm_scales(const TileMat &m, size_t tg) {
  return (const float *)(m.base + tg * m.rs + m.so);
}

// The experts of one layer.
struct ExpertLayout {
  const unsigned char *base;  // expert 0
  size_t expert_bytes;        // one expert
  size_t gu_bytes;            // one expert's gate/up records (its down records follow)
  unsigned tgc;               // codes bytes of one tile-group (64 x BPL)
  __host__ __device__ unsigned rec_gu() const { return 2 * tgc + 128; }
  __host__ __device__ unsigned rec_d() const { return tgc + 64; }
  // m = 0 gate, 1 up, 2 down
  __host__ __device__ TileMat mat(int e, int m) const {
    const unsigned char *x = base + (size_t)e * expert_bytes;
    TileMat t;
    if (m == 2) {
      t.base = x + gu_bytes;
      t.rs = rec_d();
      t.so = tgc;
    } else {
      t.base = x + (size_t)m * tgc;
      t.rs = rec_gu();
      t.so = 2 * tgc + 64 * (unsigned)m - (unsigned)m * tgc;
    }
    return t;
  }
};

__host__ __device__ inline unsigned tile_codes_bytes(int fmt) { return 64u * (fmt == 4 ? 16u : 12u); }
// gate/up and whole-expert sizes for a shape (I % 16 == 0, H % 16 == 0)
__host__ __device__ inline ExpertLayout expert_layout(const unsigned char *base, int H, int I, int fmt) {
  ExpertLayout l;
  const int ngh = (H + 127) / 128, ngi = (I + 127) / 128;
  l.base = base;
  l.tgc = tile_codes_bytes(fmt);
  l.gu_bytes = (size_t)(I / 16) * ngh * l.rec_gu();
  l.expert_bytes = l.gu_bytes + (size_t)(H / 16) * ngi * l.rec_d();
  return l;
}

}  // namespace sw
