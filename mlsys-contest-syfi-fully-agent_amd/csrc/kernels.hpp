// kernels.hpp -- launchers of the device stages (one per .hip file).
#pragma once

#include "moe_common.hpp"

namespace moe {

hipError_t launch_route(const float* logits, const uint16_t* bias, float rsf, int T, int64_t offset,
                        const Layout& L, char* ws, hipStream_t stream);
// T <= 16: GEMM1 routes the tokens itself (each workgroup, from LDS; workgroup
// 0 writes the routing results to the workspace), so no launch_route runs
// before it.  The routing inputs are unused for larger T.
bool gemm1_routes(int T);
hipError_t launch_gemm1(const uint8_t* hs, const float* hs_scale, int T, const uint8_t* w13,
                        const float* w13_scale, const float* logits, const uint16_t* bias, float rsf,
                        int64_t offset, const Layout& L, char* ws, hipStream_t stream);
// T <= kGemm2StreamMaxTokens (moe_common.hpp): GEMM2 also performs the
// weighted combine, and no combine pass runs.
bool gemm2_fuses_combine(int T);
hipError_t launch_gemm2(int T, const uint8_t* w2, const float* w2_scale, const Layout& L, char* ws, void* out,
                        hipStream_t stream);
hipError_t launch_combine(int T, const Layout& L, char* ws, void* out, hipStream_t stream);
// bf16 hidden rows -> e4m3 rows + transposed per-128-block scales.
hipError_t launch_quantize_hidden(const uint16_t* x, int T, uint8_t* q, float* scale, hipStream_t stream);

}  // namespace moe
