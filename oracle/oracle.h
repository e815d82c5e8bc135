/*
 * CPU oracle for the GGUF quantized matrix-vector path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of recipe's own
 * arithmetic for this path. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only as the checker or as
 * the timed CPU baseline. The product library never links or calls it.
 *
 * Every function cites the reference file:line it restates.
 *
 * Pinning of each function (what checks it, beyond its own formula):
 *   orc_fp16_from_f32 / orc_f32_from_fp16  exhaustive/boundary comparison with
 *        IEEE binary16 (numpy) and an exact-rational model of the subnormal
 *        truncate-then-round path (tests/test_oracle.py).
 *   orc_dequant_rows   bit-exact against ggml's textbook loop-form decoders
 *        (a different formulation, numpy), recipe's Q8_0 known answer
 *        (suite.rs:186-193), and for Q4_K the independent scalar Q4_K x Q8_1
 *        algebra of evidence/2026-10-10-m60-p2p/bench.rs:193-226.
 *   orc_matvec_f64     brute force on tiny shapes, linearity, scale-by-2.
 *   orc_matvec_recipe_f32  within 1e-6 of orc_matvec_f64, suite.rs known answer.
 *   orc_matvec_recipe_fast bit-identical to orc_matvec_recipe_f32.
 *   orc_topk           brute force with a stable sort and closed-form softmax.
 *   orc_moe_f64        a numpy composition of the block on tiny shapes.
 *   orc_q4k_q81_reference  is itself the bench.rs algorithm (a second,
 *        reference-held algorithm that pins the Q4_K decode).
 */
#ifndef RQMV_ORACLE_H
#define RQMV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids, as recipe's GGUF parser maps them (recipe.rs:9925-9961). */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q6_K = 14 };

uint16_t orc_fp16_from_f32(float value);
float orc_f32_from_fp16(uint16_t value);
void orc_fp16_from_f32_n(const float* in, uint16_t* out, size_t n);

/* Values per block and bytes per block (recipe.rs:15811-15826). 0 on unknown. */
int orc_block_values(int format);
int orc_block_bytes(int format);

/* One weight of a block in f64, as HostQuantOps runs the format's program. */
double orc_dequant_value(int format, const uint8_t* block, int index);

/* rows x cols weights (GGUF row-major blocks) decoded to float: (float)f64. */
int orc_dequant_rows(int format, const uint8_t* bytes, int64_t rows, int64_t cols, float* out);

/* y[m*ldy + n] = sum_k w[n][k] * x[m*ldx + k] in f64. */
int orc_matvec_f64(int format, const uint8_t* bytes, int64_t rows, int64_t cols, const double* x, int m_count,
                   int64_t ldx, double* y, int64_t ldy);

/* recipe's fp32 float packed path: per run (one block of 256/32 values) a
 * sequential fp32 fma chain from zero over exact fp32 weights, runs added in
 * order into the row sum. threads <= 1 runs serially; otherwise rows are
 * split contiguously over that many POSIX threads (the CPU backend's workers). */
int orc_matvec_recipe_f32(int format, const uint8_t* bytes, int64_t rows, int64_t cols, const float* x, int m_count,
                          int64_t ldx, float* y, int64_t ldy, int threads);

/* The same products as orc_matvec_recipe_f32, bit for bit, on recipe's
 * compiled schedule (block headers decoded once per block, eight rows per SIMD
 * lane group, rows split over `threads` POSIX threads): the timed CPU
 * baseline (recipe_cpu.c). Q4_0, Q8_0, Q4_K and Q6_K. */
int orc_matvec_recipe_fast(int format, const uint8_t* bytes, int64_t rows, int64_t cols, const float* x, int m_count,
                           int64_t ldx, float* y, int64_t ldy, int threads);

/* Top-k routing of one position (amd-nv-cpu.ll:4653-4716): dense weights[E],
 * zero off the kept set. scoring 0 = softmax, 1 = sigmoid. orc_topk_biased
 * chooses by probability + bias[e] (bias may be NULL: the raw score). */
int orc_topk(const double* scores, int experts, int top, int scoring, int renormalize, double* weights);
int orc_topk_biased(const double* scores, int experts, int top, int scoring, int renormalize, const double* bias,
                    double* weights);

/* recipe's activation `code` (Activation::code, recipe.rs:13925-13950; 32 =
 * Gelu under the gelu table) applied to x in f64 (activation_program,
 * recipe.rs:22579-22727); factor = Scale's constant / PReLU's slope. Returns 0
 * for an unknown code. */
int orc_activation(int code, double factor, double x, double* out);

/* The gguf_moe block at one position in f64 (recipe.rs:23386-23459):
 * router [experts x d] f16, banks [experts x hidden x d] (gate, up) and
 * [experts x d x hidden] (down) in `format`, gated by `activation`
 * (act(gate x) * up x); an optional selection bias (experts values); a shared
 * expert (hidden_shared wide) weighted by shared_gate_activation of a [d] f16
 * vector, or by one when that vector is NULL. Any of gate_sh/up_sh/down_sh
 * NULL disables the shared expert. Returns -2 for an unknown activation. */
int orc_moe_f64(int format, int d_model, int experts, int top, int hidden, int scoring, int renormalize, double scale,
                int activation, double activation_factor, const double* selection_bias, const uint16_t* router,
                const uint8_t* gate_bank, const uint8_t* up_bank, const uint8_t* down_bank, int hidden_shared,
                const uint16_t* shared_gate_vec, int shared_gate_activation, const uint8_t* gate_sh,
                const uint8_t* up_sh, const uint8_t* down_sh, const double* x, double* y, double* route_weights);

/* evidence/2026-10-10-m60-p2p/bench.rs:193-226: Q4_K rows (cols multiple of
 * 256) against x quantized to Q8_1-style records, int dots, f64 block scales.
 * Also returns the quantized activations as values (q * d) in x_used. */
int orc_q4k_q81_reference(const uint8_t* w, int64_t rows, int64_t cols, const float* x, float* y, double* x_used);

/* evidence/2026-10-10-m60-p2p/bench.rs:177-190: deterministic xorshift Q4_K
 * rows of 16 superblocks (4096 columns). */
void orc_q4k_xorshift_rows(uint32_t seed, int64_t rows, uint16_t scale_bits, uint8_t* out);

/* recipe's int(8) sum (the default profile's `sum = "int8"`, Cargo.toml:143-162,
 * and the llama.cpp profile's, Cargo.toml:182-201). recipe's GPU backends run
 * it with 32 lanes per output (a wave of 32, NVIDIA's warp or gfx11/gfx12's
 * wave32); this restatement keeps those 32 lanes as an array.
 *
 * Activation records (amd-nv-cpu.ll:1304-1500): per `step` inputs (32 or 256)
 * one fp32 step d and a signed 8-bit code per input. The step's extreme is the
 * input of largest magnitude (lane scans keep the first, the 32-lane butterfly
 * prefers the larger signed value on equal magnitudes); inverse = -127/extreme,
 * d = 1/inverse, code = clamp(roundeven(x*inverse), -128, 127); an all-zero
 * step has d = 0 and zero codes. d is stored once per 32 inputs. */
int orc_q8_records(const float* x, int64_t k, int step, float* d, int8_t* codes);

/* The int(8) product of GGUF block rows against Q8 records, per position m:
 * y[m*rows + n] in fp32. Slices of 16 values (Q4_K, Q6_K at a 32 step; Q8_0 and
 * Q4_0 at either step: build.rs:776-866, 886-915) have their ints made with
 * dot4 and their fp32 tail in the helper's order; lane l adds slices l, l+32,
 * ... in order and the lanes meet in a butterfly of offsets 16..1
 * (amd-nv-cpu.ll:1804-1836, 2031-2090, 2156-2170). At a 256 step Q4_K folds
 * whole blocks with fma in block order (amd-nv-cpu.ll:1545-1733; four
 * quarter fmas for positions m < M - M%4 unless `tail` makes the last
 * position whole) and Q6_K keeps eight fma chains (amd-nv-cpu.ll:1836-2031).
 * Inputs must be finite. */
int orc_int8_matvec(int format, const uint8_t* bytes, int64_t rows, int64_t cols, const float* x, int m_count,
                    int step, int tail, float* y);

/* IEEE binary16 encode, round half to even (LLVM's fptrunc float -> half). */
uint16_t orc_fp16_rne(float value);

/* The storage recipe's int(8) profile gives a bound weight that is not Q4_K or
 * Q8_0 (finish_int_sums + requantize_bound, recipe.rs:22327-22437): each
 * 32-value block of the decoded weight re-encoded as Q8_0 by the device
 * quantizer (recipe.rs:8016-8080): extreme = first value of largest magnitude,
 * scale = |extreme| / 127, inverse = 1 / scale (0 for a zero scale), code =
 * clamp(trunc(v * inverse + (v * inverse >= 0 ? 0.5 : -0.5)), -128, 127),
 * d = fp16(scale) rounded half to even. Sources Q4_0, Q6_K, F16 and Q8_0
 * (whose values decode exactly in fp32). out: rows * cols / 32 * 34 bytes. */
int orc_requantize_q8_0(int format, const uint8_t* bytes, int64_t rows, int64_t cols, uint8_t* out);

#ifdef __cplusplus
}
#endif
#endif
