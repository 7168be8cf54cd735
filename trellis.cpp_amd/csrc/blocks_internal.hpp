// Elementwise steps between library calls (blocks.hip), for the composite blocks. Both return a
// tsp_status and leave the message like the entry points.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace tsp {

// y[i] = x[i] (or silu(x[i])) stored as ydt: f32, or f16 / bf16 rounded to nearest even
int f32_to(const float* x, int64_t n, void* y, int ydt, bool silu, hipStream_t s);
// y[i] += x[i] for x of dtype xdt
int add_to(float* y, const void* x, int xdt, int64_t n, hipStream_t s);

}  // namespace tsp
