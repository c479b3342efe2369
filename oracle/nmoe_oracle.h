/*
 * nmoe_oracle.h -- CPU oracle for the routed-expert MoE path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library (libnmoe_hip.so)
 * links, loads or calls this code.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg use it, and only as the checker / the timed CPU
 * baseline, never as the product path.
 *
 * Every routine restates a reference routine (file:line relative to the
 * reference repository root) with the same operation order and types, or, for
 * the two reduction orders that exist only on the GPU side of this build
 * (router logits), mirrors that fixed order so identical inputs give
 * identical bits.  Build flags: -O2 -ffp-contract=off, so nothing is fused
 * unless written with fmaf().
 *
 * Pinning (see tests/): math.m routines are checked against golden vectors
 * produced by the real src/math.m compiled as C (oracle/_ref) and against
 * closed forms; the expf restatement is checked against the host libm (the
 * exhaustive check over all non-positive floats found zero mismatches);
 * the generator is checked against distribution moments and hand-computed
 * SplitMix64 values; the dispatch permutation against a brute-force sort.
 */
#ifndef NMOE_ORACLE_H
#define NMOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_HIDDEN 2048
#define ORC_INTER 512
#define ORC_EXPERTS 256
#define ORC_GROUP 64
#define ORC_MAX_K 8

/* math.m:7-19 */
float orc_bf16_to_f32(uint16_t v);
uint16_t orc_f32_to_bf16(float v);
void orc_bf16_to_f32_array(const uint16_t *in, float *out, size_t n);
void orc_f32_to_bf16_bits(const uint32_t *in, uint16_t *out, size_t n);

/* math.m:21-32 */
float orc_sigmoid(float x);
float orc_silu(float x);

/* math.m:34-65 */
void orc_rms_norm(const float *input, const uint16_t *weight_bf16, float *output, size_t count, float eps,
                  int add_one);

/* math.m:67-162 */
void orc_softmax(float *values, size_t count);
size_t orc_topk(const float *values, size_t count, size_t k, uint32_t *indices, float *selected_values);
void orc_renormalize(float *values, size_t count);
void orc_swiglu(const float *gate, const float *up, float *output, size_t count);

/* math.m:191-274 */
void orc_unpack_row(const uint32_t *packed_row, uint16_t *output, size_t in_dim, int quant_bits);
void orc_dequant_row(const uint32_t *packed_row, const uint16_t *scales_row, const uint16_t *biases_row,
                     float *output, size_t in_dim, int quant_bits);
void orc_dequant_matvec(const uint32_t *packed, const uint16_t *scales, const uint16_t *biases,
                        const float *input, float *output, size_t out_dim, size_t in_dim, int quant_bits);

/* The converter's quantiser and packer, convert_qwen36.py:147-211: bf16
 * rows [rows][in_dim] -> packed u32 [rows][in_dim*bits/32], bf16 scales and
 * biases [rows][in_dim/64].  Finite inputs. */
void orc_quantize_rows(const uint16_t *rows_bf16, int rows, int in_dim, int bits, uint32_t *packed,
                       uint16_t *scales, uint16_t *biases);

/* runtime.m:1498-1511 (softmax -> top-k -> renormalise on one token's logits).
 * idx/w are padded to 8 slots: unused slots get index 0 and weight 0
 * (kernels.metal:1767-1775).  probs (nullable) receives the softmax output.
 * Returns the number of selected experts, or -1 for k outside 1..8. */
int orc_route(const float *logits, int num_experts, int k, uint32_t *idx8, float *w8, float *probs);

/* glibc expf (sysdeps/ieee754/flt-32/e_expf.c, ARM optimized-routines method)
 * as selected on x86-64 hosts with FMA: all multiply-adds fused.  The GPU
 * softmax evaluates exactly these steps in double precision. */
float orc_expf_restated(float x);

/* Router logits, mirroring the GPU's fixed reduction order: lane L of a
 * 64-lane wave owns the 16-byte chunks L, L+64, L+128, ... of a row and
 * accumulates them sequentially with fmaf; the 64 partials are combined by
 * the balanced pairwise tree over lanes in order ((p0+p1)+(p2+p3), ...). */
void orc_router_logits_bf16(const uint16_t *w, const float *x, int num_experts, int hidden, float *out);
void orc_router_logits_q4(const uint32_t *w, const uint16_t *scales, const uint16_t *biases, const float *x,
                          int num_experts, int hidden, float *out);

/* Expert pack layout: convert_qwen36.py:38-64 == runtime.m:2240-2252,
 * sizes expert_io.m:90-99. */
size_t orc_expert_size(int bits);
void orc_expert_offsets(int bits, size_t off9[9]);

/* One expert on one token, the reference CPU way: two math.m dequant
 * matvecs + math.m SwiGLU (gate/up), one math.m dequant matvec (down). */
void orc_expert_gate_up(const uint8_t *expert, int bits, const float *x, float *act512);
void orc_expert_down(const uint8_t *expert, int bits, const float *act512, float *y2048);

/* Weighted combine, kernels.metal:1394-1423 / 1539-1541:
 * out = h_mid + sum_k w_k*y_k + sigmoid(g)*shared, moe summed in slot order.
 * shared_out / shared_gate_raw are nullable (then the term is absent). */
void orc_shared_expert(const uint32_t *gw, const uint16_t *gs, const uint16_t *gb, const uint32_t *uw,
                       const uint16_t *us, const uint16_t *ub, const uint32_t *dw, const uint16_t *ds,
                       const uint16_t *db, const uint32_t *sw, const uint16_t *ss, const uint16_t *sb, const float *x,
                       float *shared_out, float *shared_gate_raw);
void orc_combine(const float *h_mid, const float *y, const float *w, int k, const float *shared_out,
                 const float *shared_gate_raw, float *out, int hidden);

/* Full decode step for ntok tokens (tokens are independent).
 * x: fp32 [ntok][2048]; router bf16 [256][2048]; layer_pack = 256 experts.
 * idx/w out: [ntok][8]. act (nullable): [ntok][8][512]. */
int orc_moe_step_bf16router(const uint8_t *layer_pack, int bits, const uint16_t *router_w, const float *x,
                            int ntok, int k, const float *h_mid, const float *shared_out,
                            const float *shared_gate_raw, float *out, uint32_t *idx, float *w, float *logits,
                            float *act);

/* One token through one layer with its input RMSNorm (math.m:34-65, unit
 * weight): x = RMSNorm(h_in); h_out = h_in + MoE(x).  idx/w/x_out nullable. */
int orc_moe_layer_rmsnorm(const uint8_t *layer_pack, int bits, const uint16_t *router_w, const float *h_in, float eps,
                          int k, float *h_out, uint32_t *idx8, float *w8, float *x_out);

/* One token through one layer's MoE block in the reference's order
 * (runtime.m:3144-3201, 2908-2999): post-attention RMSNorm (weighted or
 * unit), router (kind 0 bf16, 1 q4), routing, optional shared expert (12
 * pointers: gate w/s/b, up w/s/b, down w/s/b, score w/s/b), experts,
 * combine, optional next-layer input RMSNorm.  See nmoe_oracle.c. */
int orc_moe_block(const uint8_t *layer_pack, int bits, int router_kind, const uint16_t *router_bf16,
                  const uint32_t *rq_w, const uint16_t *rq_s, const uint16_t *rq_b, const void *const *shared,
                  const uint16_t *post_norm, int add_one, const float *h_mid, float eps, int k, float *out,
                  const uint16_t *next_norm, float *next_x, uint32_t *idx8, float *w8, float *x_out);

/* Experts only (routing given): idx/w [ntok][8]. */
int orc_moe_experts(const uint8_t *layer_pack, int bits, const float *x, int ntok, int k, const uint32_t *idx,
                    const float *w, const float *h_mid, const float *shared_out, const float *shared_gate_raw,
                    float *out, float *act);

/* Dispatch permutation for batched / prefill: stable counting sort of the
 * routed rows r = t*k + s by expert idx[t*stride + s]; ties keep r order.
 * perm[ntok*k], offsets[num_experts+1]. */
void orc_dispatch(const uint32_t *idx, int ntok, int k, int stride, int num_experts, uint32_t *perm,
                  uint32_t *offsets);

/* Synthetic data generator (counter-based SplitMix64).  The device generator
 * in the library implements the same definition. */
uint64_t orc_syn_mix64(uint64_t z);
uint64_t orc_syn_stream(uint64_t seed, uint32_t layer, uint32_t expert, uint32_t tag);
uint64_t orc_syn_rand64(uint64_t stream, uint64_t i);
float orc_syn_normal(uint64_t stream, uint64_t i);
void orc_syn_expert(uint8_t *dst, int bits, uint64_t seed, uint32_t layer, uint32_t expert, float sigma);
void orc_syn_layer(uint8_t *dst, int bits, uint64_t seed, uint32_t layer, float sigma);
void orc_syn_bf16_normal(uint16_t *dst, size_t n, uint64_t seed, uint32_t layer, uint32_t tag, float sigma);

#ifdef __cplusplus
}
#endif

#endif
