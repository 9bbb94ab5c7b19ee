// Internal: the persistent batch-1 decode kernel over a stack of layers
// (moe_stack.hip) and what the rest of the library calls of it.
#pragma once

#include <stddef.h>

#include "shiftwing_moe.h"

namespace sw {

constexpr int kStackMaxE = 1024;    // experts per layer
constexpr int kStackMaxK = 16;      // routes per token
constexpr int kStackMaxIsh = 4096;  // shared intermediate (integer-sum block size)

// Whether the persistent kernel takes layers of this shape on this device.
bool stack_shape_ok(const ColiCuda *ctx, const ColiMoeShape &s);
// One token through layers[0..n) (all of one shape): y + l*ys = layer l of
// x + l*xs.  Returns 0 on success, -1 on error, 1 when the shape is outside
// the kernel's limits (the caller takes another path).
int stack_step(ColiCuda *ctx, ColiMoeLayer *const *layers, int n, float *y, size_t ys, const float *x, size_t xs,
               int *route_idx, float *route_weight);
// -1 (with the error text set) when a previous stack call aborted.
int stack_check_abort(ColiCuda *ctx);
void stack_release(ColiCuda *ctx);

}  // namespace sw
