// Library-internal fused nn op, for the GPT forward.
#pragma once

namespace bmb {

// res_out = a + b (residual_forward), then ln_out, mean, rstd =
// layernorm(res_out) (layernorm_forward), in one pass over the rows: the same
// fp32 results as the two launches of src/gpt.cu:266-268,278-283. Null stream.
void residual_layernorm_forward(float *res_out, float *ln_out, float *mean, float *rstd,
                                const float *a, const float *b, const float *weight,
                                const float *bias, int N, int C);

}  // namespace bmb
