// grad.h — per-row gradients shared by the gradient passes and the training
// walk (compute_gradients, Shaders.swift:96-138 and the objectives'
// additions).  Device code only.
#pragma once
#include <math.h>

#include "mbk.h"

namespace mbk {

__device__ __forceinline__ float clampf(float x, float lo, float hi) {
    return fminf(fmaxf(x, lo), hi);
}

// exp evaluated in double and rounded to float once; the oracle does the same.
__device__ __forceinline__ float exp_via_double(float x) { return (float)exp((double)x); }

// (g, h) of one row for objective `obj` (Shaders.swift:105-135).
__device__ __forceinline__ void row_grad(const GradParams &gp, float f, float y, float w, float &g,
                                         float &h) {
    switch (gp.objective) {
    case 1: {
        float q = 1.0f / (1.0f + exp_via_double(-f));
        float ww = y > 0.5f ? gp.aux : 1.0f;
        g = (q - y) * ww;
        h = fmaxf(q * (1.0f - q), 1e-6f) * ww;
        break;
    }
    case 2: g = f > y ? 1.0f : -1.0f; h = 1.0f; break;
    case 3: g = clampf(f - y, -gp.alpha, gp.alpha); h = 1.0f; break;
    case 4: g = f > y ? (1.0f - gp.alpha) : -gp.alpha; h = 1.0f; break;
    case 5: {
        float mu = exp_via_double(clampf(f, -30.0f, 30.0f));
        g = mu - y; h = fmaxf(mu, 1e-6f);
        break;
    }
    case 6: {
        float fc = clampf(f, -30.0f, 30.0f);
        float e2 = exp_via_double((2.0f - gp.aux) * fc), e1 = exp_via_double((1.0f - gp.aux) * fc);
        g = e2 - y * e1;
        h = fmaxf((2.0f - gp.aux) * e2 - (1.0f - gp.aux) * y * e1, 1e-6f);
        break;
    }
    default: g = f - y; h = 1.0f; break;
    }
    if (gp.has_weights) { g *= w; h *= w; }
}

}  // namespace mbk
