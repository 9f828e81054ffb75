/*
 * GPT-2 model: allocation, initialisation, forward, backward -- C-ABI drop-in
 * for bare-metal-bard's src/gpt.h, running on this library's gfx950 kernels
 * (gemm.h, flash.h, attention.h, nn.h).
 *
 * The structs have the reference's fields, names and order (src/gpt.h:10-67),
 * so a caller such as the trainer or the gradient checker reads g.acts.losses,
 * g.params_mem, g.num_params, ... exactly as before. The functions take a
 * pointer in C; the C++ view adds the reference's reference-taking overloads
 * (gpt_alloc(g), gpt_forward(g, x, y), ...).
 *
 * Memory (src/gpt.cu:73-185): four parameter-sized buffers (params, grads,
 * AdamW m and v), one arena of forward activations for all layers, one arena
 * of single-layer backward scratch, and token/target buffers. With
 * use_flash the attention keeps only lse (B, NH, T) per layer; otherwise the
 * unfused path keeps qkvr (4BTC) and att (B, NH, T, T) per layer.
 * All kernels run on the null stream.
 */
#ifndef BMB_GPT_H
#define BMB_GPT_H

#include <stddef.h>
#ifndef __cplusplus
#include <stdbool.h>
#endif

#ifdef __cplusplus
extern "C" {
#endif
/* Only the declarations below are exported from libbmb.so (built with -fvisibility=hidden). */
#pragma GCC visibility push(default)

/* src/gpt.h:10-17 */
typedef struct GPTConfig {
    int max_seq_len;  /* T */
    int vocab_size;   /* V, the real number of distinct tokens */
    int padded_vocab; /* Vp >= V; logits and wte carry Vp rows/columns */
    int n_layer;      /* L */
    int n_head;       /* NH */
    int n_embd;       /* C */
} GPTConfig;

enum { NUM_PARAM_TENSORS = 16 };

/* src/gpt.h:21-25 */
typedef struct Parameters {
    float *wte, *wpe;
    float *ln1w, *ln1b, *qkvw, *qkvb, *attprojw, *attprojb;
    float *ln2w, *ln2b, *fcw, *fcb, *fcprojw, *fcprojb;
    float *lnfw, *lnfb;
} Parameters;

/* src/gpt.h:28-36 */
typedef struct Activations {
    float *encoded;
    float *ln1, *ln1_mean, *ln1_rstd;
    float *qkv, *qkvr, *att, *atty, *attproj;
    float *lse;
    float *residual2, *ln2, *ln2_mean, *ln2_rstd;
    float *fch, *fch_gelu, *fcproj, *residual3;
    float *lnf, *lnf_mean, *lnf_rstd;
    float *logits, *probs, *losses;
} Activations;

/* src/gpt.h:39-46 */
typedef struct Gradients {
    float *dres;
    float *dln1, *dln2, *datty;
    float *dqkv, *dqkvr, *datt;
    float *dsum;
    float *dfch, *dfch_gelu;
    float *dlogits, *dlnf;
} Gradients;

/* src/gpt.h:48-67. Set config, use_flash, B and T before gpt_alloc. */
typedef struct GPT {
    GPTConfig config;
    bool use_flash;
    int B, T;

    Parameters params, grads;
    size_t psize[NUM_PARAM_TENSORS];
    size_t num_params;
    float *params_mem, *grads_mem, *m_mem, *v_mem;

    Activations acts;
    Gradients gr;
    float *acts_mem, *grads_act_mem;
    size_t num_acts, num_grad_acts;

    int *d_tokens, *d_targets;
} GPT;

/* src/gpt.h:76-77 */
extern const char *const PARAM_NAMES[NUM_PARAM_TENSORS];
void param_sizes(size_t *s, const GPTConfig *c);

/* src/gpt.h:69: allocates everything listed above (device memory; AdamW
 * moments and targets zeroed). On an allocation failure it prints the
 * request and calls exit(1), as the reference's CUDA_CHECK does. */
void gpt_alloc(GPT *g);
/* src/gpt.h:70: N(0, 0.02) weights from std::mt19937(seed) and
 * std::normal_distribution<float>, the two residual projections at
 * 0.02/sqrt(2L), layernorm weights 1, biases 0 (src/gpt.cu:189-222). */
void gpt_init(GPT *g, unsigned seed);
/* src/gpt.h:73: tokens and targets are HOST arrays of B*T ids; returns the
 * mean cross-entropy loss, or 0 when targets is NULL (logits only). A token
 * id outside [0, padded_vocab) is reported on stderr and NaN is returned
 * with nothing launched; a target outside [0, padded_vocab) gives that
 * position a NaN loss (nn.h). */
float gpt_forward(GPT *g, const int *tokens, const int *targets);
/* src/gpt.h:74: gradients of the last gpt_forward with targets, written
 * (not accumulated) into grads_mem. */
void gpt_backward(GPT *g);
/* Not in the reference (its trainer never frees): releases every buffer
 * gpt_alloc made and clears the pointers. */
void gpt_free(GPT *g);

/* The GPT1 checkpoint (src/train_gpt.cu:175-227), little-endian: int magic
 * 0x47505431 ("GPT1"), the 6 ints of GPTConfig, int nvocab, nvocab bytes of
 * the character vocabulary (itos), then num_params fp32 parameters in
 * parameter order. Both return 0 on success and -1 on any I/O or format
 * error (with a message on stderr). gpt_load_checkpoint sets g->config and
 * g->T = max_seq_len from the file, then calls gpt_alloc (so set g->B and
 * g->use_flash first, on a GPT that holds no allocation) and uploads the
 * parameters; it stores up to itos_cap vocabulary bytes in itos and the full
 * count in *nvocab. */
int gpt_save_checkpoint(const GPT *g, const char *path, const char *itos, int nvocab);
int gpt_load_checkpoint(GPT *g, const char *path, char *itos, int itos_cap, int *nvocab);

/* A training step is the trainer's sequence (src/train_gpt.cu:395-460):
 * gpt_forward, gpt_backward, grad_global_norm and adamw_update (nn.h). */

#pragma GCC visibility pop
#ifdef __cplusplus
}  /* extern "C" */

/* The reference's C++ signatures (src/gpt.h:69-77). */
inline void param_sizes(size_t *s, const GPTConfig &c) { param_sizes(s, &c); }
inline void gpt_alloc(GPT &g) { gpt_alloc(&g); }
inline void gpt_init(GPT &g, unsigned seed) { gpt_init(&g, seed); }
inline float gpt_forward(GPT &g, const int *tokens, const int *targets) {
    return gpt_forward(&g, tokens, targets);
}
inline void gpt_backward(GPT &g) { gpt_backward(&g); }
inline void gpt_free(GPT &g) { gpt_free(&g); }
#endif

#endif
