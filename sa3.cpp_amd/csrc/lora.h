// Internal API of lora.hip beyond the C ABI: a group of bf16-precision adapted linears whose
// adapter-derived terms are refreshed together (one launch per stage for the whole group).
#pragma once

#include "gemm.h"

namespace sa3k {

struct LinGroup;

// lins: bf16-precision linears with bf16 working copies, all of rank `rank` (> 0); A/B/mag/bnsq
// are the device adapter pointers of each (mag/bnsq for dora), fixed for the group's lifetime.
LinGroup* lin_group_create(sa3k_ctx* ctx, sa3k_lin* const* lins, int n, const float* const* A, const float* const* B,
                           const float* const* mag, const float* const* bnsq, float scale, int dora);
// the grouped equivalent of sa3k_lin_prepare on every member
void lin_group_prepare(sa3k_ctx* ctx, LinGroup* g);
void lin_group_free(LinGroup* g);

}  // namespace sa3k
