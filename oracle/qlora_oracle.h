/*
 * qlora_oracle.h -- CPU restatement of stuarch/VkQLoRA.rs `qlora-core`.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the checker that the HIP library is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product path never does.
 *
 * Every function restates one reference function with the same loop order
 * and the same f32 rounding sequence (built with -ffp-contract=off, no
 * fast-math).  Citations are to files under the reference tree.
 */
#ifndef QLORA_ORACLE_H
#define QLORA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* qlora-core/src/quant.rs:27-50 */
extern const float OR_NF4_LEVELS[16];
#define OR_NF4_ZERO_CODE 7
#define OR_DOUBLE_QUANT_BLOCK 256

/* qlora-core/tests/quant.rs:6-24 -- xorshift64* and Box-Muller. */
typedef struct { uint64_t s; } or_rng;
double or_rng_next_f64(or_rng *r);
float or_rng_next_normal(or_rng *r);
void or_fill_normal(uint64_t *state, float *out, size_t n, float scale);
void or_fill_uniform(uint64_t *state, float *out, size_t n, float lo, float hi);

/* quant.rs:263-278 */
uint8_t or_nearest_nf4_code(float w, float absmax);

/* quant.rs:104-154 + 283-299.  codes: ceil(n/2) bytes (zeroed here).
 * double_quant == 0: scales_f32 gets ceil(n/bs) floats.
 * double_quant != 0: scale_codes gets ceil(n/bs) bytes, absmax gets
 * ceil(nb/256) floats.  Returns 0, or -1 for block_size == 0. */
int or_quantize(const float *w, size_t n, size_t block_size, int double_quant,
                uint8_t *codes, float *scales_f32, uint8_t *scale_codes,
                float *absmax);

/* quant.rs:212-221 -- decoded per-block scales. */
void or_block_scales_dq(const uint8_t *scale_codes, const float *absmax,
                        size_t nb, float *out);

/* quant.rs:157-167 -- dequantize with already-decoded block scales. */
void or_dequantize(const uint8_t *codes, const float *scales, size_t n,
                   size_t block_size, float *out);

/* lora.rs:129-183 */
void or_matmul(const float *a, const float *b, size_t m, size_t k, size_t n,
               float *c);
void or_matmul_trans_a(const float *a, const float *b, size_t m, size_t k,
                       size_t n, float *c);
void or_matmul_trans_b(const float *a, const float *b, size_t m, size_t k,
                       size_t n, float *c);

/* qlora.rs:86-107 (+ lora.rs:86-103).  w_deq is the dequantized weight
 * (out_dim x in_dim).  lora_a/lora_b may be NULL (no adapter). */
void or_qlora_forward(const float *w_deq, size_t out_dim, size_t in_dim,
                      const float *lora_a, const float *lora_b, size_t r,
                      float alpha, const float *x, size_t batch, float *y);

/* qlora.rs:116-165.  grad_a/grad_b ignored without an adapter. */
void or_qlora_backward(const float *w_deq, size_t out_dim, size_t in_dim,
                       const float *lora_a, const float *lora_b, size_t r,
                       float alpha, const float *x, const float *dy,
                       size_t batch, float *grad_x, float *grad_a,
                       float *grad_b);

/* optim.rs:32-249 -- paged 8-bit Adam. */
typedef struct or_adam or_adam;
or_adam *or_adam_create(float lr, float beta1, float beta2, float eps,
                        size_t block_size, size_t max_resident_pages);
void or_adam_destroy(or_adam *o);
/* Returns pages_streamed, or (size_t)-1 on a length mismatch. */
size_t or_adam_step(or_adam *o, float **params, const float *const *grads,
                    const size_t *lens, size_t count);
size_t or_adam_state_bytes(const or_adam *o);
/* optim.rs:84-100 */
float or_quantize_block_i8(const float *x, size_t len, uint8_t *codes);
void or_dequant_block_i8(const uint8_t *codes, float absmax, size_t len,
                         float *out);
/* Read back the int8 state of parameter `idx` (for state-level parity). */
int or_adam_get_state(const or_adam *o, size_t idx, uint8_t *m_codes,
                      float *m_scales, uint8_t *v_codes, float *v_scales,
                      uint64_t *step);

/* ---- qlora-model glue around the projections (qlora-model/src/llama.rs) */
/* rmsnorm_in_place (llama.rs:730-739): y = x * (1/sqrt(mean(x^2)+eps)) * w
 * per row of h; y may alias x. */
void or_rmsnorm(const float *x, const float *w, size_t rows, size_t h,
                float eps, float *y);
/* rmsnorm_backward (llama.rs:605-628): dx (rows x h) and dw (h). */
void or_rmsnorm_backward(const float *x, const float *w, const float *dy,
                         size_t rows, size_t h, float eps, float *dx,
                         float *dw);
/* silu / sigmoid / silu_prime (llama.rs:516-527). */
float or_silu(float x);
float or_silu_prime(float x);
/* MLP activation (llama.rs:452-456): act = silu(gate) * up. */
void or_swiglu(const float *gate, const float *up, size_t n, float *act);
/* Its backward (llama.rs:559-562): dg = d_act*up*silu'(gate),
 * du = d_act*silu(gate). */
void or_swiglu_backward(const float *gate, const float *up,
                        const float *d_act, size_t n, float *dg, float *du);
/* softmax_cross_entropy (llama.rs:487-514): mean loss over seq rows and
 * dlogits (seq x vocab).  Returns the loss. */
float or_softmax_cross_entropy(const float *logits, const uint32_t *targets,
                               size_t seq, size_t vocab, float *dlogits);

#ifdef __cplusplus
}
#endif
#endif
