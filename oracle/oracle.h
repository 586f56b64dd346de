/*
 * oracle.h -- CPU oracle for the FP8 block-scale DeepSeek-V3 MoE layer
 * (moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048).
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links this code.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it,
 * and only as the checker (or, for the baseline, as the thing timed on CPU).
 *
 * Two parts:
 *   - synth_*: the deterministic input generator.  It uses integer hashing,
 *     IEEE-exact fp32 mul/div and integer-coded rounding only, so its GPU twin
 *     (the package's csrc/synth.hip) produces the same bytes.
 *   - orc_*: a plain-C restatement of the contest reference
 *     full-agent-pipeline/references/moe.py (routing, dequantisation,
 *     per-expert GEMM1 -> SwiGLU -> GEMM2, weighted accumulation, bf16 cast).
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Fixed geometry of the definition (moe.py:65-76, moe.py:16-23). */
#define ORC_H 7168
#define ORC_I 2048
#define ORC_2I 4096
#define ORC_E_LOCAL 32
#define ORC_E_GLOBAL 256
#define ORC_TOP_K 8
#define ORC_N_GROUP 8
#define ORC_TOPK_GROUP 4
#define ORC_GROUP_SIZE 32
#define ORC_BLOCK 128
#define ORC_NH_BLK 56  /* H/128  */
#define ORC_NI_BLK 16  /* I/128  */
#define ORC_N2I_BLK 32 /* 2I/128 */

/* ---- scalar formats (exact; exhaustively tested) ---------------------- */
float orc_e4m3_to_f32(uint8_t v);      /* OCP float8_e4m3fn decode           */
uint8_t orc_f32_to_e4m3(float x);      /* RNE, saturate finite to +-448      */
float orc_bf16_to_f32(uint16_t v);
uint16_t orc_f32_to_bf16(float x);     /* RNE (torch .to(bfloat16))          */
float orc_exp_f32(float x);            /* float(exp(double(x)))              */

/* ---- generator ------------------------------------------------------ */
/* Stream ids keep the five tensors independent for one seed. */
enum { SYN_LOGITS = 1, SYN_BIAS = 2, SYN_HIDDEN = 3, SYN_W13 = 4, SYN_W2 = 5 };

uint64_t synth_hash(uint64_t seed, uint32_t stream, uint64_t idx);
float synth_normal(uint64_t seed, uint32_t stream, uint64_t idx); /* ~N(0,1) */

/* logits [T,256] fp32, N(0,1); row-prefix stable in T. */
void synth_logits(uint64_t seed, int64_t T, float* out);
/* bias [256] bf16 bits, N(0,0.1) plus `hot_add` on the listed expert ids. */
void synth_bias(uint64_t seed, const int32_t* hot_ids, int n_hot, float hot_add,
                uint16_t* out);
/* hidden [T,7168] e4m3 + scales [56,T] (absmax/448 per (token,128 cols)). */
void synth_hidden(uint64_t seed, int64_t T, uint8_t* q, float* scale);
/* gemm1 weights [32,4096,7168] e4m3 + scales [32,32,56]; experts [e0,e1). */
void synth_w13(uint64_t seed, int e0, int e1, uint8_t* q, float* scale);
/* gemm2 weights [32,7168,2048] e4m3 + scales [32,56,16]; experts [e0,e1). */
void synth_w2(uint64_t seed, int e0, int e1, uint8_t* q, float* scale);

/* ---- activation quantiser (the step before the layer) ------------------ */
/* bf16 hidden rows [T,7168] -> e4m3 [T,7168] + transposed scales [56,T]:
 * scale = absmax/448 over the block's non-NaN |x| (1 if that is 0),
 * q = orc_f32_to_e4m3(x / scale).  The convention of synth_hidden, applied
 * to given values.  No counterpart in the reference (it consumes the result,
 * moe.py:32-33). */
void orc_quantize_hidden(const uint16_t* x, int64_t T, uint8_t* q, float* scale);

/* ---- routing (moe.py:123-158) ---------------------------------------- */
/* For each token: the 8 selected global expert ids sorted ascending, their
 * combination weights, and (optional) the fp32 sigmoid / biased scores.
 * Selection (including exact ties) follows torch.topk on CPU. */
void orc_route(const float* logits, const uint16_t* bias, int64_t T, float rsf,
               int32_t* ids /*[T,8]*/, float* w /*[T,8]*/,
               float* s_out /*[T,256] or NULL*/, float* sb_out /*[T,256] or NULL*/);

/* ---- full layer (moe.py:56-202) --------------------------------------- */
/* Computes output rows for `n_tok` tokens listed in `tokens` (NULL = all T).
 * out: [n_tok, 7168] bf16 bits.  dequant_all != 0 materialises fp32 copies of
 * all 32 experts' weights first, as moe.py:107-118 does (used for CPU-baseline
 * timing); otherwise only the rows of experts that are used are dequantised,
 * on the fly.  Returns 0, or -1 on allocation failure. */
int orc_moe(const float* logits, const uint16_t* bias, const uint8_t* hs,
            const float* hs_scale, const uint8_t* w13, const float* w13_scale,
            const uint8_t* w2, const float* w2_scale, int64_t local_expert_offset,
            float rsf, int64_t T, const int32_t* tokens, int64_t n_tok,
            uint16_t* out, int dequant_all);

/* Intermediate for kernel-level checks: C = silu(G1[:, I:]) * G1[:, :I] for the
 * (token, local expert) pairs given, as fp32 [n_pairs, 2048], and O = C . W2^T
 * as fp32 [n_pairs, 7168] (either may be NULL). */
int orc_expert_rows(const uint8_t* hs, const float* hs_scale, int64_t T,
                    const uint8_t* w13, const float* w13_scale, const uint8_t* w2,
                    const float* w2_scale, const int32_t* pair_token,
                    const int32_t* pair_local_expert, int64_t n_pairs, float* c_out,
                    float* o_out);

int orc_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
