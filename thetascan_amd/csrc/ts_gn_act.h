// Hidden nonlinearities of the GN fast network (device side), shared by the
// fused GN write / read kernels and the per-row activation kernel:
// sigma(pre), sigma'(pre) and the backward term sigma' dh + sigma'' dsp.
// relu2 and silu are the reference's (src/thetascan/_core/ops/nonlin.py:9-31);
// tanh is this library's extension.
#pragma once

#include <hip/hip_runtime.h>

#include "thetascan_hip.h"

namespace ts {

// sigma(pre); the slope sp = sigma'(pre) is written as a function of h =
// sigma(pre) for relu2 (2 sqrt(h) = 2 relu(pre)) and tanh (1 - h^2).
__device__ __forceinline__ float gn_sigmoid(float pre) { return 1.f / (1.f + __expf(-pre)); }
__device__ __forceinline__ float gn_act(int act, float pre) {
  if (act == TS_GN_TANH) return tanhf(pre);
  if (act == TS_GN_SILU) return pre * gn_sigmoid(pre);
  const float rp = fmaxf(pre, 0.f);
  return rp * rp;
}
// sigma'(pre): from h for relu2 and tanh, from pre for SiLU
// (silu' = sg (1 + pre (1 - sg)), sg = sigmoid(pre)).
__device__ __forceinline__ float gn_slope(int act, float pre, float hval) {
  if (act == TS_GN_SILU) {
    const float sg = gn_sigmoid(pre);
    return sg * (1.f + pre * (1.f - sg));
  }
  return act == TS_GN_TANH ? 1.f - hval * hval : 2.f * sqrtf(hval);
}
// d pre of a term dh * h + dsp * sp: sigma'(pre) dh + sigma''(pre) dsp
// (relu2: 2 relu(pre) dh + 2 dsp for pre > 0, else 0;
//  tanh: (1 - h^2) dh - 2 h (1 - h^2) dsp;
//  silu: silu'' = sg (1 - sg) (2 + pre (1 - 2 sg))).
__device__ __forceinline__ float gn_dpre(int act, float pre, float hval, float dh, float dsp) {
  if (act == TS_GN_TANH) {
    const float d1 = 1.f - hval * hval;
    return d1 * dh - 2.f * hval * d1 * dsp;
  }
  if (act == TS_GN_SILU) {
    const float sg = gn_sigmoid(pre);
    const float d1 = sg * (1.f + pre * (1.f - sg));
    const float d2 = sg * (1.f - sg) * (2.f + pre * (1.f - 2.f * sg));
    return d1 * dh + d2 * dsp;
  }
  return pre > 0.f ? 2.f * fmaxf(pre, 0.f) * dh + 2.f * dsp : 0.f;
}

}  // namespace ts
