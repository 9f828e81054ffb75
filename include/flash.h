/*
 * Fused causal multi-head attention, forward and backward -- C-ABI drop-in for
 * bare-metal-bard's src/flash.h.
 *
 * Buffer shapes (src/flash.h:29-35), all fp32, caller-owned device memory:
 *   qkv  (B, T, 3C)   fused QKV projection output, [q|k|v] along 3C,
 *                     head h at column offset h*hs, hs = C / NH
 *   out  (B, T, C)
 *   lse  (B, NH, T)   natural-log log-sum-exp of each row's scaled scores
 *   dqkv (B, T, 3C)   written, not accumulated
 *   dsum (B, NH, T)   backward scratch: rowsum(dout * out)
 * scale = 1/sqrt(hs). The T x T score matrix is never materialised. Launches
 * go to the null stream. Supported head sizes: 32, 64, 128.
 *
 * Memory: the default backward config stores the causal 32x32 tiles of dS
 * (fp32, 4 KiB each, B*NH*n(n+1)/2 of them with n = ceil(T/32)) in a
 * workspace that each call leases from a library-owned pool of the device
 * and returns once it has queued its work; the pool keeps its buffers for
 * reuse until the process ends and holds as many as were ever leased at once
 * (one per concurrently calling host thread), however many threads come and
 * go. All of it runs on the null stream, where launches from every host
 * thread run in submission order, so the next call to lease a buffer runs
 * after the last one that used it. If it cannot be allocated the backward
 * falls back to a config that recomputes S and dP instead and allocates
 * nothing; flash_attention_backward_cfg can select such a config directly.
 * The same configs run as persistent
 * workgroups on a per-shape work plan that the first backward call of a
 * shape computes on the host and uploads (a few KB per pass, kept per device
 * until the process ends): that first call therefore makes two small
 * allocations and two synchronous copies. Likewise the default forward
 * config, when its whole grid fits on the device at once, places its work
 * by a per-shape order that its first call of a shape uploads (4 bytes per
 * workgroup: one small allocation and one synchronous copy).
 */
#ifndef BMB_FLASH_H
#define BMB_FLASH_H

#ifndef __cplusplus
#include <stdbool.h>
#endif

#ifdef __cplusplus
extern "C" {
#endif
/* Only the declarations below are exported from libbmb.so (built with -fvisibility=hidden). */
#pragma GCC visibility push(default)

/* src/flash.h:36-37. Runs the default config, then any legal config; if none
 * fits the head size, prints a message and calls exit(1) like the reference
 * (src/flash.cu:419-432). */
void flash_attention_forward(float *out, float *lse, const float *qkv, int B,
                             int T, int C, int NH);

/* src/flash.h:39-41. Same fallback rule (src/flash.cu:988-1003). */
void flash_attention_backward(float *dqkv, float *dsum, const float *dout,
                              const float *qkv, const float *out,
                              const float *lse, int B, int T, int C, int NH);

/* Tuning harness, src/flash.h:48-53: configs are enumerated and named; the
 * _cfg entry returns false (launching nothing) for an unknown id, a head size
 * the config cannot serve, or a shape it cannot run. */
int flash_num_configs(void);
const char *flash_config_name(int cfg);
int flash_default_config(void);
bool flash_attention_forward_cfg(int cfg, float *out, float *lse,
                                 const float *qkv, int B, int T, int C, int NH);

/* src/flash.h:56-62 */
int flash_num_bwd_configs(void);
const char *flash_bwd_config_name(int cfg);
int flash_default_bwd_config(void);
bool flash_attention_backward_cfg(int cfg, float *dqkv, float *dsum,
                                  const float *dout, const float *qkv,
                                  const float *out, const float *lse, int B,
                                  int T, int C, int NH);

#pragma GCC visibility pop
#ifdef __cplusplus
}
#endif
#endif
