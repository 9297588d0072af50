// Internal launchers shared between translation units of libaltxs_hip.so.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

hipError_t altxs_launch_cdf(const float* in, int64_t rows, int V, int flags, bool from_logits,
                            float* probs, uint32_t* cum, hipStream_t s);

// Row-parallel softmax -> CDF (no renormalisation); V % 64 == 0.  The chunked
// form reads the LM head's per-64-column tile statistics.
// Whether altxs_launch_cdf_stats uses one workgroup per row for this shape
// (it then forms the row statistics itself and does not read stats).
bool altxs_cdf_rows_kernel(int64_t rows, int V);
// xcd_rows (row kernel, rows % 64 == 0): row tile t of 8 rows on XCD t % 8.
hipError_t altxs_launch_cdf_stats(const float* logits, const float2* stats, int64_t rows, int V,
                                  float* probs, uint32_t* cum, hipStream_t s, bool xcd_rows = false);

struct AltxsAttnArgs;
hipError_t altxs_launch_attn(const AltxsAttnArgs& a, hipStream_t s);
// The same decode launch also forming the out-projection's per-head terms
// (o_part[(r * H + h) * o_n + n], before the group scales); hipErrorInvalidValue
// for the shapes it does not cover (W = 1, MHA, tiled bf16 cache, bf16
// operands and output, o_bits in {2, 3, 4, 6}, o_n % 16 == 0, o_n <= 512).
hipError_t altxs_launch_attn_o(const AltxsAttnArgs& a, const uint8_t* o_codes, int o_bits, int o_n,
                               float* o_part, hipStream_t s);
