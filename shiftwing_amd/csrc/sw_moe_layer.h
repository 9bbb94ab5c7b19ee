// Internal: the HBM-resident layer object behind ColiMoeLayer and the
// decode-step entry shared by moe.hip and moe_decode.hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include "shiftwing_moe.h"
#include "sw_expert_layout.h"

struct ColiMoeLayer {
  ColiMoeShape sh;               // the device shape: I and shared I rounded up to the tiles (16, 64)
  int I_src, Ish_src;            // the caller's I and shared I (rows past them hold zeros)
  int src_fmt;                   // the caller's expert format: 2 (int2 rows, widened to the int4 records), 3, 4
  int ngh, ngi;                  // groups along H (gate/up cols) and I (down cols)
  float *router;                 // [E][H]
  float *sgate_row;              // [H]
  signed char *sh_gq, *sh_uq, *sh_dq;  // row-major int8
  float *sh_gs, *sh_us, *sh_ds;
  unsigned char *experts;        // routed experts' records (sw_expert_layout.h)
  sw::ExpertLayout xl;           // ... and where they lie
  unsigned long long *stats;     // device [2]: tokens, exact fallbacks
  // decode-step fan-in counters and int32 accumulators, owned by the layer
  // (zeroed at creation and returned to zero by every step), so a context
  // serving layers of different shapes never sees another layer's state
  unsigned *sync;
  size_t sync_words;
  int router_mode;
  size_t bytes;
  void *alloc[16];
  int nalloc;
};

namespace sw {
// words of ColiMoeLayer::sync for a layer shape
size_t decode_sync_words(const ColiMoeShape &s);
// One routed expert given in container format src_fmt (the layer's own; 2 or
// 4 in a layer held as int4 records)
int set_expert_as(ColiCuda *ctx, ColiMoeLayer *L, int expert, int src_fmt, const unsigned char *gq, const float *gs,
                  const unsigned char *uq, const float *us, const unsigned char *dq, const float *ds);
// One decoded token through one layer (three kernels).  Returns 0 on success,
// -1 on error, 1 when the layer shape is outside the decode kernels' limits.
int decode_step(ColiCuda *ctx, ColiMoeLayer *L, float *y, const float *x, int *route_idx, float *route_weight);
}  // namespace sw
