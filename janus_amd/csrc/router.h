// Internal interface of the router kernels (router.hip).
#pragma once

#include "common.h"

namespace janus {

struct RouteWorkspace {
  float* partial;  // [k ranges, T, padded E] approximate-logit partial sums
  float2* xstat;   // [k ranges, T] (||x||^2, x . w_shared_gate) partial sums
};

size_t router_prep_bytes(int E, int H);
size_t route_workspace_bytes(int T, int H, int E);
RouteWorkspace carve_route(Carver& c, int T, int H, int E);
int check_route_sizes(int T, int H, int E, int top_k);
// valid [T] (nonzero = a real token) or null: a padding token gets expert id E (dropped by align), weight 0, gate 0.
int launch_route(const uint16_t* x, const float* w, const void* prep, const float* bias, const uint16_t* wsg, int T,
                 int H, int E, int top_k, const uint8_t* valid, int32_t* topk_idx, float* topk_w, float* gamma,
                 const RouteWorkspace& ws, hipStream_t stream);

}  // namespace janus
