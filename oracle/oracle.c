/*
 * CPU oracle for the GGUF quantized matrix-vector path: TEST INFRASTRUCTURE.
 * Used only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
 * as the checker or as the timed restatement of recipe's CPU path. Never part
 * of the product path. The declarations in oracle.h list what pins each function.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* recipe.rs:15098-15113 `fp16`: round half to even on normal values; values
 * that become subnormal are first truncated to the subnormal grid scaled by
 * 2^13 and then rounded; finite values at or beyond 2^16 map to inf when their
 * mantissa is zero and to a NaN (0x7c01) otherwise, exactly as written there. */
uint16_t orc_fp16_from_f32(float value) {
    uint32_t bits;
    memcpy(&bits, &value, 4);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    int32_t exponent = (int32_t)((bits >> 23) & 0xffu) - 112;
    uint32_t mantissa = bits & 0x7fffffu;
    if (exponent <= 0) {
        if (exponent < -10) return sign;
        uint32_t v = (mantissa | 0x800000u) >> (1 - exponent);
        return (uint16_t)(sign | ((v + 0xfffu + ((v >> 13) & 1u)) >> 13));
    }
    if (exponent >= 31) return (uint16_t)(sign | 0x7c00u | (mantissa != 0 ? 1u : 0u));
    uint32_t rounded = mantissa + 0xfffu + ((mantissa >> 13) & 1u);
    if (rounded & 0x800000u) {
        int32_t e = exponent + 1 < 31 ? exponent + 1 : 31;
        return (uint16_t)(sign | ((uint32_t)e << 10));
    }
    return (uint16_t)(sign | ((uint32_t)exponent << 10) | (rounded >> 13));
}

/* recipe.rs:15114-15126 `unfp16`. */
float orc_f32_from_fp16(uint16_t value) {
    uint32_t sign = ((uint32_t)value & 0x8000u) << 16;
    uint32_t exponent = (value >> 10) & 31u;
    uint32_t mantissa = value & 1023u;
    uint32_t bits;
    if (exponent == 0) {
        if (mantissa == 0) {
            bits = sign;
        } else {
            uint32_t shift = (uint32_t)__builtin_clz(mantissa) - 21u;
            bits = sign | ((113u - shift) << 23) | ((mantissa << (shift + 13u)) & 0x7fffffu);
        }
    } else if (exponent == 31) {
        bits = sign | 0x7f800000u | (mantissa << 13);
    } else {
        bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

void orc_fp16_from_f32_n(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_fp16_from_f32(in[i]);
}

/* recipe.rs:15811-15826 (the quantizations! table rows for these formats). */
int orc_block_values(int format) {
    switch (format) {
        case ORC_F32: case ORC_F16: return 1;
        case ORC_Q4_0: case ORC_Q8_0: return 32;
        case ORC_Q4_K: case ORC_Q6_K: return 256;
        default: return 0;
    }
}

int orc_block_bytes(int format) {
    switch (format) {
        case ORC_F32: return 4;
        case ORC_F16: return 2;
        case ORC_Q4_0: return 18;
        case ORC_Q8_0: return 34;
        case ORC_Q4_K: return 144;
        case ORC_Q6_K: return 210;
        default: return 0;
    }
}

/* HostQuantOps::half (recipe.rs:4006-4008 via `half`, recipe.rs:15130). */
static double half_at(const uint8_t* b, int offset) {
    return (double)orc_f32_from_fp16((uint16_t)(b[offset] | (b[offset + 1] << 8)));
}

/* dequant_scalar, Q8_0 (recipe.rs:3782-3833, man 8, variant 0, header 2):
 * the code is the sign-extended byte 2 + i, times the fp16 scale at 0. */
static double dequant_q8_0(const uint8_t* b, int i) {
    int64_t code = (int8_t)b[2 + i];
    return (double)code * half_at(b, 0);
}

/* dequant_scalar, Q4_0 (man 4, sign 1, variant 0): nibble (i / 16) of byte
 * 2 + i % 16, less 1 << (man - sign) = 8, times the scale at 0. */
static double dequant_q4_0(const uint8_t* b, int i) {
    uint64_t byte = b[2 + (i % 16)];
    uint64_t code = (byte >> (4 * (i / 16))) & 15u;
    int64_t signed_code = (int64_t)(code - 8u);
    return (double)signed_code * half_at(b, 0);
}

/* dequant_q45k with man = 4 (recipe.rs:3687-3741): nibble (sub % 2) of byte
 * 16 + 32 * (sub / 2) + i % 32; 6-bit scale and minimum of sub-block `sub`
 * by the k_scale packing (recipe.rs:15204-15210); w = d*sc*q - dmin*m. */
static double dequant_q4_k(const uint8_t* b, int i) {
    uint64_t sub = (uint64_t)i / 32, within = (uint64_t)i % 32;
    uint64_t packed = b[16 + (sub / 2) * 32 + within];
    uint64_t code = (packed >> ((sub % 2) * 4)) & 15u;
    uint64_t low_scale = b[sub + 4] & 63u;
    uint64_t low_minimum = b[sub + 8] & 63u;
    uint64_t high_packed = b[sub + 8];
    uint64_t high_scale = (high_packed & 15u) | ((uint64_t)(b[sub] >> 6) << 4);
    uint64_t high_minimum = (high_packed >> 4) | ((uint64_t)(b[sub + 4] >> 6) << 4);
    uint64_t scale_code = sub < 4 ? low_scale : high_scale;
    uint64_t minimum_code = sub < 4 ? low_minimum : high_minimum;
    double step = half_at(b, 0) * (double)scale_code;
    double base = half_at(b, 2) * (double)minimum_code;
    double product = step * (double)code;
    return product - base;
}

/* dequant_q6k (recipe.rs:3743-3780). */
static double dequant_q6_k(const uint8_t* b, int i) {
    uint64_t chunk = (uint64_t)i / 128, local = (uint64_t)i % 128;
    uint64_t group = local / 32, within = local % 32;
    uint64_t low = b[chunk * 64 + within + 32 * (group & 1u)];
    uint64_t high = b[chunk * 32 + within + 128];
    uint64_t low_bits = (low >> (4 * (group / 2))) & 15u;
    uint64_t high_bits = ((high >> (2 * group)) & 3u) << 4;
    int64_t code = (int64_t)((low_bits | high_bits) - 32u);
    int64_t factor = (int8_t)b[192 + chunk * 8 + group * 2 + within / 16];
    double scaled = half_at(b, 208) * (double)factor;
    return scaled * (double)code;
}

double orc_dequant_value(int format, const uint8_t* block, int index) {
    switch (format) {
        case ORC_F32: {
            float f;
            memcpy(&f, block, 4);
            return (double)f;
        }
        case ORC_F16: return half_at(block, 0);
        case ORC_Q4_0: return dequant_q4_0(block, index);
        case ORC_Q8_0: return dequant_q8_0(block, index);
        case ORC_Q4_K: return dequant_q4_k(block, index);
        case ORC_Q6_K: return dequant_q6_k(block, index);
        default: return NAN;
    }
}

static int shape_ok(int format, int64_t rows, int64_t cols) {
    int bv = orc_block_values(format);
    return bv > 0 && rows >= 0 && cols > 0 && cols % bv == 0;
}

/* decode_blocks with HostQuantOps (recipe.rs:16141-16157, 3973-4057). */
int orc_dequant_rows(int format, const uint8_t* bytes, int64_t rows, int64_t cols, float* out) {
    if (!shape_ok(format, rows, cols)) return -1;
    const int bv = orc_block_values(format), bb = orc_block_bytes(format);
    const int64_t blocks = rows * (cols / bv);
    for (int64_t blk = 0; blk < blocks; ++blk) {
        const uint8_t* b = bytes + blk * bb;
        for (int i = 0; i < bv; ++i) out[blk * bv + i] = (float)orc_dequant_value(format, b, i);
    }
    return 0;
}

int orc_matvec_f64(int format, const uint8_t* bytes, int64_t rows, int64_t cols, const double* x, int m_count,
                   int64_t ldx, double* y, int64_t ldy) {
    if (!shape_ok(format, rows, cols) || m_count <= 0) return -1;
    const int bv = orc_block_values(format), bb = orc_block_bytes(format);
    const int64_t nb = cols / bv;
    double* w = (double*)malloc(sizeof(double) * (size_t)cols);
    if (!w) return -2;
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t blk = 0; blk < nb; ++blk)
            for (int i = 0; i < bv; ++i)
                w[blk * bv + i] = orc_dequant_value(format, bytes + (r * nb + blk) * bb, i);
        for (int m = 0; m < m_count; ++m) {
            double s = 0.0;
            const double* xm = x + (int64_t)m * ldx;
            for (int64_t k = 0; k < cols; ++k) s += w[k] * xm[k];
            y[(int64_t)m * ldy + r] = s;
        }
    }
    free(w);
    return 0;
}

/* recipe.rs:3216-3218 `dot_run`: a run is a whole block of 32 or more values,
 * or 32 values of smaller blocks. */
static int dot_run(int format) {
    int bv = orc_block_values(format);
    return bv >= 32 ? bv : 32;
}

typedef struct {
    int format;
    const uint8_t* bytes;
    int64_t cols, row_begin, row_end;
    const float* x;
    int m_count;
    int64_t ldx, ldy;
    float* y;
} recipe_job;

/* emit_run_decoder (recipe.rs:7880-7903): per run, `sum = fma(weight, input,
 * sum)` for j = 0..run from zero; packed_lanes_body (amd-nv-cpu.ll:3053-3088):
 * run parts added in order into the row sum, stored in fp32. The weight is the
 * state-type decode, which equals (float) of the f64 decode for these formats. */
static void* recipe_rows(void* arg) {
    const recipe_job* job = (const recipe_job*)arg;
    const int format = job->format;
    const int bv = orc_block_values(format), bb = orc_block_bytes(format);
    const int run = dot_run(format);
    const int64_t nb = job->cols / bv;
    float* w = (float*)malloc(sizeof(float) * (size_t)run);
    float* total = (float*)malloc(sizeof(float) * (size_t)job->m_count);
    for (int64_t r = job->row_begin; r < job->row_end; ++r) {
        for (int m = 0; m < job->m_count; ++m) total[m] = 0.0f;
        for (int64_t k0 = 0; k0 < job->cols; k0 += run) {
            for (int j = 0; j < run; ++j) {
                int64_t k = k0 + j;
                const uint8_t* b = job->bytes + (r * nb + k / bv) * bb;
                w[j] = (float)orc_dequant_value(format, b, (int)(k % bv));
            }
            for (int m = 0; m < job->m_count; ++m) {
                const float* xm = job->x + (int64_t)m * job->ldx + k0;
                float part = 0.0f;
                for (int j = 0; j < run; ++j) part = fmaf(w[j], xm[j], part);
                total[m] = total[m] + part;
            }
        }
        for (int m = 0; m < job->m_count; ++m) job->y[(int64_t)m * job->ldy + r] = total[m];
    }
    free(w);
    free(total);
    return NULL;
}

int orc_matvec_recipe_f32(int format, const uint8_t* bytes, int64_t rows, int64_t cols, const float* x, int m_count,
                          int64_t ldx, float* y, int64_t ldy, int threads) {
    if (!shape_ok(format, rows, cols) || m_count <= 0 || cols % dot_run(format) != 0) return -1;
    if (threads <= 1 || rows < 2) {
        recipe_job job = {format, bytes, cols, 0, rows, x, m_count, ldx, ldy, y};
        recipe_rows(&job);
        return 0;
    }
    if (threads > rows) threads = (int)rows;
    pthread_t* tids = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    recipe_job* jobs = (recipe_job*)malloc(sizeof(recipe_job) * (size_t)threads);
    int64_t per = rows / threads, extra = rows % threads, begin = 0;
    for (int t = 0; t < threads; ++t) {
        int64_t count = per + (t < extra ? 1 : 0);
        recipe_job job = {format, bytes, cols, begin, begin + count, x, m_count, ldx, ldy, y};
        jobs[t] = job;
        begin += count;
        pthread_create(&tids[t], NULL, recipe_rows, &jobs[t]);
    }
    for (int t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
    free(tids);
    free(jobs);
    return 0;
}

/* @sigmoid (amd-nv-cpu.ll:5007-5009): 1 / (1 + exp(-x)). */
static double sigmoid_ref(double x) { return 1.0 / (1.0 + exp(-x)); }

/* @topk_score (amd-nv-cpu.ll:4486-4488). */
static double topk_score(double score, double maximum, int sigmoid) {
    return sigmoid ? sigmoid_ref(score) : exp(score - maximum);
}

/* @topk_forward_body (amd-nv-cpu.ll:4653-4716): repeated scans pick the
 * highest unmarked key, the lower expert on a tie (a strict greater-than over
 * ascending ids). The key (@topk_key, amd-nv-cpu.ll:4653-4660) is the raw
 * score without a selection bias; with one it is the expert's probability
 * (its sigmoid, or its softmax over every expert: exp(score - max) / total,
 * the maximum and total taken over all experts first) plus its bias. The
 * weights come from the unbiased scores: the maximum and total run over the
 * kept set when renormalizing, over every expert otherwise; softmax (or
 * renormalized sigmoid) divides by the total. */
int orc_topk_biased(const double* scores, int experts, int top, int scoring, int renormalize, const double* bias,
                    double* weights) {
    if (experts <= 0 || top <= 0 || top > experts) return -1;
    const int sigmoid = scoring != 0, renorm = renormalize != 0;
    const int every = !renorm, divide = renorm || !sigmoid;
    double all_max = 0.0;
    for (int e = 0; e < experts; ++e)
        if (e == 0 || scores[e] > all_max) all_max = scores[e];
    double all_total = 0.0;
    for (int e = 0; e < experts; ++e) all_total = all_total + topk_score(scores[e], all_max, sigmoid);
    for (int e = 0; e < experts; ++e) weights[e] = 0.0;
    for (int pick = 0; pick < top; ++pick) {
        int best = -1;
        double best_score = 0.0;
        for (int c = 0; c < experts; ++c) {
            int unmarked = weights[c] == 0.0;
            double key = scores[c];
            if (bias) {
                const double raw = topk_score(scores[c], all_max, sigmoid);
                key = (sigmoid ? raw : raw / all_total) + bias[c];
            }
            int better = best == -1 || key > best_score;
            if (unmarked && better) {
                best = c;
                best_score = key;
            }
        }
        weights[best] = 1.0;
    }
    double maximum = 0.0;
    int first = 1;
    for (int m = 0; m < experts; ++m) {
        int member = weights[m] == 1.0 || every;
        if (member && (first || scores[m] > maximum)) {
            maximum = scores[m];
            first = 0;
        }
    }
    double total = 0.0;
    for (int s = 0; s < experts; ++s) {
        int member = weights[s] == 1.0 || every;
        total = total + (member ? topk_score(scores[s], maximum, sigmoid) : 0.0);
    }
    double denominator = divide ? total : 1.0;
    for (int w = 0; w < experts; ++w) {
        int marked = weights[w] == 1.0;
        weights[w] = marked ? topk_score(scores[w], maximum, sigmoid) / denominator : 0.0;
    }
    return 0;
}

int orc_topk(const double* scores, int experts, int top, int scoring, int renormalize, double* weights) {
    return orc_topk_biased(scores, experts, top, scoring, renormalize, NULL, weights);
}

/* fp16 rounding of an f64 value (RNE, as the Half scalar op rounds the GELU
 * table's input and output), back to f64. */
static double half_round(double v) { return (double)orc_f32_from_fp16(orc_fp16_rne((float)v)); }

/* Activation::code() values (recipe.rs:13925-13950). */
enum {
    ACT_LINEAR = 0, ACT_COS = 1, ACT_EXP = 2, ACT_LOG = 3, ACT_LN = 4, ACT_HUBER = 5, ACT_TAN = 6, ACT_RELU = 7,
    ACT_LEAK = 8, ACT_SIGMOID = 9, ACT_TANH = 10, ACT_SELU = 11, ACT_GELU = 12, ACT_SILU = 13, ACT_ELU = 14,
    ACT_PRELU = 15, ACT_SCALE = 16, ACT_SQRT = 17, ACT_SOFTPLUS = 18, ACT_GELU_FP16 = 32
};

/* recipe's activation programs (activation_program, recipe.rs:22579-22727)
 * in f64, with the default constants of Cargo.toml:117-124 (leak slope 0.01,
 * ELU alpha 1, SELU alpha/scale, GELU scale sqrt(2/pi) and cubic 0.044715,
 * Huber threshold 1). `factor` is Scale's constant and PReLU's slope.
 * ACT_GELU_FP16 is Gelu under the llama.cpp profile's gelu table (its input
 * and result rounded to fp16 inside (-10, 10); the input itself at 10 and
 * above, zero at -10 and below). Returns 0 for an unknown code. */
int orc_activation(int code, double factor, double x, double* out) {
    const double one = 1.0, half = 0.5;
    const int positive = x > 0.0;
    double r;
    switch (code) {
        case ACT_LINEAR: r = x; break;
        case ACT_COS: r = cos(x); break;
        case ACT_EXP: r = exp(x); break;
        case ACT_SQRT: r = sqrt(x); break;
        case ACT_SOFTPLUS: r = (positive ? x : 0.0) + log(one + exp(0.0 - fabs(x))); break;
        case ACT_LOG:
        case ACT_LN: {
            const double magnitude = log(one + fabs(x));
            const double signed_ = positive ? magnitude : 0.0 - magnitude;
            r = code == ACT_LOG ? signed_ / 2.302585092994045684 : signed_;
            break;
        }
        case ACT_HUBER: {
            const double t = 1.0, a = fabs(x);
            r = a > t ? t * (a - half * t) : half * (x * x);
            break;
        }
        case ACT_TAN: r = sin(x) / cos(x); break;
        case ACT_RELU: r = positive ? x : 0.0; break;
        case ACT_LEAK: r = positive ? x : 0.01 * x; break;
        case ACT_PRELU: r = positive ? x : factor * x; break;
        case ACT_ELU:
        case ACT_SELU: {
            const double alpha = code == ACT_SELU ? 1.6732632423543772 : 1.0;
            const double masked = positive ? 0.0 : x;
            const double negative = alpha * (exp(masked) - one);
            r = positive ? x : negative;
            if (code == ACT_SELU) r = 1.0507009873554805 * r;
            break;
        }
        case ACT_SIGMOID: r = half * (tanh(half * x) + one); break;
        case ACT_SILU: r = x * (half * (tanh(half * x) + one)); break;
        case ACT_TANH: r = tanh(x); break;
        case ACT_GELU: r = (half * x) * (one + tanh((0.7978845608028654 * x) * fma(0.044715 * x, x, one))); break;
        case ACT_GELU_FP16: {
            if (x > 10.0) {
                r = x;
            } else if (x < -10.0) {
                r = 0.0;
            } else {
                const double h = half_round(x);
                r = half_round((half * h) * (one + tanh((0.7978845608028654 * h) * fma(0.044715 * h, h, one))));
            }
            break;
        }
        case ACT_SCALE: r = factor * x; break;
        default: return 0;
    }
    *out = r;
    return 1;
}

static double act_apply(int code, double factor, double x) {
    double r = NAN;
    orc_activation(code, factor, x, &r);
    return r;
}

static double row_dot_f64(int format, const uint8_t* row_bytes, int64_t cols, const double* x) {
    const int bv = orc_block_values(format), bb = orc_block_bytes(format);
    double s = 0.0;
    for (int64_t k = 0; k < cols; ++k) s += orc_dequant_value(format, row_bytes + (k / bv) * bb, (int)(k % bv)) * x[k];
    return s;
}

static int64_t row_bytes_of(int format, int64_t cols) {
    return cols / orc_block_values(format) * orc_block_bytes(format);
}

/* One gated expert (recipe.rs:23386-23401 lower_experts + lower_gated,
 * 23279-23286): out += weight * down(act(gate x) * up x). */
static void expert_add(int format, int d, int hidden, const uint8_t* gate, const uint8_t* up, const uint8_t* down,
                       int activation, double factor, const double* x, double weight, double* h, double* out) {
    const int64_t in_row = row_bytes_of(format, d), out_row = row_bytes_of(format, hidden);
    for (int f = 0; f < hidden; ++f) {
        double g = row_dot_f64(format, gate + f * in_row, d, x);
        double u = row_dot_f64(format, up + f * in_row, d, x);
        h[f] = act_apply(activation, factor, g) * u;
    }
    for (int n = 0; n < d; ++n) out[n] += weight * row_dot_f64(format, down + n * out_row, hidden, h);
}

/* lower_gguf_moe (recipe.rs:23415-23459): router contraction over f16 weights,
 * TopK (with the selection bias when given), routed scale, the routed experts
 * in ascending id, then the shared expert added: weighted by its gate's
 * activation of a [d] f16 vector when gated (SharedExpert::Gated), by one
 * when not (SharedExpert::Ungated). */
int orc_moe_f64(int format, int d_model, int experts, int top, int hidden, int scoring, int renormalize, double scale,
                int activation, double activation_factor, const double* selection_bias, const uint16_t* router,
                const uint8_t* gate_bank, const uint8_t* up_bank, const uint8_t* down_bank, int hidden_shared,
                const uint16_t* shared_gate_vec, int shared_gate_activation, const uint8_t* gate_sh,
                const uint8_t* up_sh, const uint8_t* down_sh, const double* x, double* y, double* route_weights) {
    if (!shape_ok(format, 1, d_model) || !shape_ok(format, 1, hidden)) return -1;
    double probe;
    if (!orc_activation(activation, activation_factor, 0.5, &probe) ||
        !orc_activation(shared_gate_activation, activation_factor, 0.5, &probe))
        return -2;
    double* scores = (double*)malloc(sizeof(double) * (size_t)experts);
    double* weights = (double*)malloc(sizeof(double) * (size_t)experts);
    int hmax = hidden > hidden_shared ? hidden : hidden_shared;
    double* h = (double*)malloc(sizeof(double) * (size_t)(hmax > 0 ? hmax : 1));
    for (int e = 0; e < experts; ++e) {
        double s = 0.0;
        for (int k = 0; k < d_model; ++k) s += (double)orc_f32_from_fp16(router[(int64_t)e * d_model + k]) * x[k];
        scores[e] = s;
    }
    int rc = orc_topk_biased(scores, experts, top, scoring, renormalize, selection_bias, weights);
    if (rc == 0) {
        for (int n = 0; n < d_model; ++n) y[n] = 0.0;
        const int64_t bank_in = (int64_t)hidden * row_bytes_of(format, d_model);
        const int64_t bank_out = (int64_t)d_model * row_bytes_of(format, hidden);
        for (int e = 0; e < experts; ++e) {
            weights[e] *= scale;
            if (weights[e] == 0.0) continue;
            expert_add(format, d_model, hidden, gate_bank + e * bank_in, up_bank + e * bank_in,
                       down_bank + e * bank_out, activation, activation_factor, x, weights[e], h, y);
        }
        if (route_weights)
            for (int e = 0; e < experts; ++e) route_weights[e] = weights[e];
        if (gate_sh && up_sh && down_sh && hidden_shared > 0) {
            double weight = 1.0;
            if (shared_gate_vec) {
                double g = 0.0;
                for (int k = 0; k < d_model; ++k) g += (double)orc_f32_from_fp16(shared_gate_vec[k]) * x[k];
                weight = act_apply(shared_gate_activation, activation_factor, g);
            }
            double* shared = (double*)calloc((size_t)d_model, sizeof(double));
            expert_add(format, d_model, hidden_shared, gate_sh, up_sh, down_sh, activation, activation_factor, x,
                       weight, h, shared);
            for (int n = 0; n < d_model; ++n) y[n] = y[n] + shared[n];
            free(shared);
        }
    }
    free(scores);
    free(weights);
    free(h);
    return rc;
}

/* evidence/2026-10-10-m60-p2p/bench.rs:193-226, generalised from 4096 columns
 * to any multiple of 256. */
int orc_q4k_q81_reference(const uint8_t* w, int64_t rows, int64_t cols, const float* x, float* y, double* x_used) {
    if (cols <= 0 || cols % 256 != 0) return -1;
    const int64_t nblk = cols / 32, nsb = cols / 256;
    int32_t* q = (int32_t*)calloc((size_t)cols, sizeof(int32_t));
    double* d = (double*)calloc((size_t)nblk, sizeof(double));
    for (int64_t b = 0; b < nblk; ++b) {
        float mx = 0.0f;
        for (int l = 0; l < 32; ++l) mx = fmaxf(mx, fabsf(x[b * 32 + l]));
        float raw_d = mx / 127.0f;
        if (mx == 0.0f) continue;
        uint32_t bits;
        memcpy(&bits, &raw_d, 4);
        int e = (int)((bits >> 23) & 255u) - 127;
        int p = e - 10 > -24 ? e - 10 : -24;
        float step = ldexpf(1.0f, p);
        d[b] = (double)(nearbyintf(raw_d / step) * step); /* round half to even in the default mode */
        for (int l = 0; l < 32; ++l) q[b * 32 + l] = (int32_t)roundf(x[b * 32 + l] / raw_d);
    }
    if (x_used)
        for (int64_t k = 0; k < cols; ++k) x_used[k] = (double)q[k] * d[k / 32];
    for (int64_t row = 0; row < rows; ++row) {
        double acc = 0.0;
        for (int64_t sb = 0; sb < nsb; ++sb) {
            const uint8_t* blk = w + (row * nsb + sb) * 144;
            double wd = (double)orc_f32_from_fp16((uint16_t)(blk[0] | (blk[1] << 8)));
            double wm = (double)orc_f32_from_fp16((uint16_t)(blk[2] | (blk[3] << 8)));
            for (int sub = 0; sub < 8; ++sub) {
                int scale, mn;
                if (sub < 4) {
                    scale = blk[4 + sub] & 63;
                    mn = blk[8 + sub] & 63;
                } else {
                    scale = (blk[12 + sub - 4] & 15) | ((blk[4 + sub - 4] >> 6) << 4);
                    mn = (blk[12 + sub - 4] >> 4) | ((blk[8 + sub - 4] >> 6) << 4);
                }
                int32_t dot = 0, sum = 0;
                for (int lane = 0; lane < 32; ++lane) {
                    uint8_t packed = blk[16 + (sub / 2) * 32 + lane];
                    int weight = (sub & 1) == 0 ? (packed & 15) : (packed >> 4);
                    int32_t a = q[sb * 256 + sub * 32 + lane];
                    dot += weight * a;
                    sum += a;
                }
                acc += ((double)(scale * dot) * wd - (double)(mn * sum) * wm) * d[sb * 8 + sub];
            }
        }
        y[row] = (float)acc;
    }
    free(q);
    free(d);
    return 0;
}

/* evidence/2026-10-10-m60-p2p/bench.rs:177-190. */
void orc_q4k_xorshift_rows(uint32_t seed, int64_t rows, uint16_t scale_bits, uint8_t* out) {
    uint32_t state = seed;
    const int64_t blocks = rows * 16;
    for (int64_t blk = 0; blk < blocks; ++blk) {
        uint8_t* b = out + blk * 144;
        b[0] = (uint8_t)(scale_bits & 0xff);
        b[1] = (uint8_t)(scale_bits >> 8);
        b[2] = b[0];
        b[3] = b[1];
        for (int i = 0; i < 4; ++i) {
            b[4 + i] = (uint8_t)(1 + ((state >> (i * 2)) % 3));
            b[8 + i] = (uint8_t)(1 + ((state >> (i * 3)) % 3));
        }
        for (int i = 0; i < 4; ++i)
            b[12 + i] = (uint8_t)((1 + ((state >> (i * 2)) % 3)) | ((1 + ((state >> (i * 3)) % 3)) << 4));
        for (int j = 16; j < 144; ++j) {
            state ^= state << 13;
            state ^= state >> 17;
            state ^= state << 5;
            b[j] = (uint8_t)state;
        }
    }
}

/* ---- recipe's int(8) sum ---------------------------------------------------
 * Restated from amd-nv-cpu.ll (contraction_forward_gemv_wave_body, 1231-2241)
 * and the slice helpers build.rs:743-915, with recipe's 32 GPU lanes kept as
 * arrays. fp32 throughout; the Makefile builds without contraction, so every
 * product and sum below rounds on its own, and fmaf is the state's madd. */

#define ORC_LANES 32

/* amd-nv-cpu.ll:1469-1470: the partner replaces the lane's extreme when its
 * magnitude is larger, or equal with a larger signed value. */
static int q8_partner_wins(float partner, float own) {
    const float ap = fabsf(partner), ao = fabsf(own);
    return ap > ao || (ap == ao && partner > own);
}

/* amd-nv-cpu.ll:1408-1500. */
int orc_q8_records(const float* x, int64_t k, int step, float* d, int8_t* codes) {
    if (k <= 0 || k % 32 != 0 || (step != 32 && step != 256)) return -1;
    const int64_t blocks = k / 32, span = step / 32;
    for (int64_t g0 = 0; g0 < blocks; g0 += span) {
        const int64_t g1 = g0 + span < blocks ? g0 + span : blocks;
        float lane[ORC_LANES], next[ORC_LANES];
        for (int v = 0; v < ORC_LANES; ++v) {
            float acc = 0.0f;
            for (int64_t b = g0; b < g1; ++b) {
                const float value = x[b * 32 + v];
                if (fabsf(value) > fabsf(acc)) acc = value;
            }
            lane[v] = acc;
        }
        for (int off = ORC_LANES / 2; off > 0; off >>= 1) {
            for (int v = 0; v < ORC_LANES; ++v)
                next[v] = q8_partner_wins(lane[v ^ off], lane[v]) ? lane[v ^ off] : lane[v];
            memcpy(lane, next, sizeof lane);
        }
        const float extreme = lane[0];
        const int nonzero = fabsf(extreme) > 0.0f;
        const float safe = nonzero ? extreme : 1.0f;
        const float inverse_raw = -127.0f / safe;
        const float d_raw = 1.0f / inverse_raw;
        const float inverse = nonzero ? inverse_raw : 0.0f;
        const float step_d = nonzero ? d_raw : 0.0f;
        for (int64_t b = g0; b < g1; ++b) {
            d[b] = step_d;
            for (int v = 0; v < 32; ++v) {
                const float scaled = x[b * 32 + v] * inverse;
                int code = (int)nearbyintf(scaled); /* round half to even in the default mode */
                if (code < -128) code = -128;
                if (code > 127) code = 127;
                codes[b * 32 + v] = (int8_t)code;
            }
        }
    }
    return 0;
}

static float f16_at(const uint8_t* p) { return orc_f32_from_fp16((uint16_t)(p[0] | (p[1] << 8))); }

/* get_scale_min_k4 as amd-nv-cpu's slice helper reads it (build.rs:817). */
static void q4k_scale_min(const uint8_t* blk, int g, int* sc, int* m) {
    const uint8_t* s = blk + 4;
    if (g < 4) {
        *sc = s[g] & 63;
        *m = s[g + 4] & 63;
    } else {
        *sc = (s[g + 4] & 15) | ((s[g - 4] >> 6) << 4);
        *m = (s[g + 4] >> 4) | ((s[g] >> 6) << 4);
    }
}

/* Slice l (0..15) of a Q4_K block: codes of sub-block l/2, values 16*(l&1)..+16.
 * rc: the block's 256 codes; ints only (build.rs:817-845). */
static void q4k_slice_ints(const uint8_t* blk, const int8_t* rc, int l, int32_t* dot, int32_t* sum) {
    const int g = l >> 1, h = l & 1, shift = (g & 1) * 4;
    const uint8_t* q = blk + 16 + (g >> 1) * 32 + h * 16;
    const int8_t* c = rc + g * 32 + h * 16;
    int32_t dt = 0, sm = 0;
    for (int i = 0; i < 16; ++i) {
        dt += ((q[i] >> shift) & 15) * c[i];
        sm += c[i];
    }
    *dot = dt;
    *sum = sm;
}

/* build.rs:845-848: the fp32 tail of a Q4_K slice. rd: the block's 8 record steps. */
static float q4k_slice(const uint8_t* blk, const float* rd, const int8_t* rc, int l) {
    int32_t dot, sum;
    int sc, m;
    q4k_slice_ints(blk, rc, l, &dot, &sum);
    q4k_scale_min(blk, l >> 1, &sc, &m);
    const float group_d = f16_at(blk) * (float)sc;
    const float group_dmin = f16_at(blk + 2) * (float)m;
    const float dot_scaled = group_d * (float)dot;
    const float minimum_scaled = group_dmin * (float)sum;
    const float value = dot_scaled - minimum_scaled;
    return rd[l >> 1] * value;
}

/* Q6_K code n (0..255) of a block (build.rs:893-899 field positions). */
static int q6k_code(const uint8_t* blk, int n) {
    const int chunk = n / 128, local = (n % 128) / 32, within = n % 32;
    const int lo = (blk[chunk * 64 + (local & 1) * 32 + within] >> ((local >> 1) * 4)) & 15;
    const int hi = (blk[128 + chunk * 32 + within] >> (local * 2)) & 3;
    return lo | (hi << 4);
}

/* build.rs:886-915: a Q6_K slice; the scale index is the slice index. */
static float q6k_slice(const uint8_t* blk, const float* rd, const int8_t* rc, int l) {
    int32_t dot = 0, sum = 0;
    for (int i = 0; i < 16; ++i) {
        dot += q6k_code(blk, l * 16 + i) * rc[l * 16 + i];
        sum += rc[l * 16 + i];
    }
    const int32_t dot_signed = dot - sum * 32;
    const float scaled = (float)(int8_t)blk[192 + l] * (float)dot_signed;
    const float value = rd[l >> 1] * scaled;
    return f16_at(blk + 208) * value;
}

/* build.rs:776-804: slice h (0, 1) of a Q8_0 or Q4_0 block against its record
 * (rd: the record's step, rc: its 32 codes). Q4_0 takes the low nibbles for
 * slice 0 and the high ones for slice 1 and subtracts 8 times the code sum;
 * the minimum term is zero for both formats. */
static float b32_slice(int format, const uint8_t* blk, float rd, const int8_t* rc, int h) {
    int32_t dot = 0, sum = 0;
    for (int i = 0; i < 16; ++i) {
        const int c = rc[h * 16 + i];
        const int w = format == 8 ? (int)(int8_t)blk[2 + h * 16 + i] : (blk[2 + i] >> (4 * h)) & 15;
        dot += w * c;
        sum += c;
    }
    if (format == 2) dot -= sum * 8;
    const float d = f16_at(blk);
    const float minimum = 0.0f;
    const float dot_scaled = d * (float)dot;
    const float minimum_scaled = minimum * (float)sum;
    const float value = dot_scaled + minimum_scaled;
    return rd * value;
}

/* amd-nv-cpu.ll:2156-2170: the lanes' butterfly, offsets 16..1; lane 0's value. */
static float lanes_reduce(float* lane) {
    float next[ORC_LANES];
    for (int off = ORC_LANES / 2; off > 0; off >>= 1) {
        for (int v = 0; v < ORC_LANES; ++v) next[v] = lane[v] + lane[v ^ off];
        memcpy(lane, next, sizeof next);
    }
    return lane[0];
}

/* One row of 16-value slices: lane l adds slices l, l+32, ... in order
 * (amd-nv-cpu.ll:1804-1836 Q4_K, 2011-2031 Q6_K, 2055-2090 Q8_0 / Q4_0). */
static float row_slices(int format, const uint8_t* row, int64_t cols, const float* rd, const int8_t* rc) {
    float lane[ORC_LANES];
    for (int v = 0; v < ORC_LANES; ++v) lane[v] = 0.0f;
    const int64_t slices = cols / 16;
    for (int64_t s = 0; s < slices; ++s) {
        float value;
        if (format == 12) {
            const int64_t b = s / 16;
            value = q4k_slice(row + b * 144, rd + b * 8, rc + b * 256, (int)(s % 16));
        } else if (format == 14) {
            const int64_t b = s / 16;
            value = q6k_slice(row + b * 210, rd + b * 8, rc + b * 256, (int)(s % 16));
        } else {
            const int64_t b = s / 2;
            value = b32_slice(format, row + b * orc_block_bytes(format), rd[b], rc + b * 32, (int)(s % 2));
        }
        lane[s % ORC_LANES] = lane[s % ORC_LANES] + value;
    }
    return lanes_reduce(lane);
}

/* amd-nv-cpu.ll:1545-1733: Q4_K under a 256 step. Each slice's ints are the
 * group scale times its dot and the group minimum times its code sum
 * (build.rs:861-866); the four quarters' ints (four slices each) are exact.
 * whole: one fma per block with the block's int; otherwise one per quarter. */
static float row_q4k_256(const uint8_t* row, int64_t cols, const float* rd, const int8_t* rc, int whole) {
    float acc = 0.0f, accmin = 0.0f;
    for (int64_t b = 0; b < cols / 256; ++b) {
        const uint8_t* blk = row + b * 144;
        int32_t dq[4] = {0, 0, 0, 0}, mq[4] = {0, 0, 0, 0};
        for (int l = 0; l < 16; ++l) {
            int32_t dot, sum;
            int sc, m;
            q4k_slice_ints(blk, rc + b * 256, l, &dot, &sum);
            q4k_scale_min(blk, l >> 1, &sc, &m);
            dq[l >> 2] += sc * dot;
            mq[l >> 2] += m * sum;
        }
        const float d8 = rd[b * 8];
        const float scale = f16_at(blk) * d8;
        const float dscale = f16_at(blk + 2) * d8;
        if (whole) {
            const int32_t dot_all = (dq[0] + dq[1]) + (dq[2] + dq[3]);
            const int32_t min_all = (mq[0] + mq[1]) + (mq[2] + mq[3]);
            acc = fmaf((float)dot_all, scale, acc);
            accmin = fmaf((float)min_all, dscale, accmin);
        } else {
            for (int q = 0; q < 4; ++q) {
                acc = fmaf((float)dq[q], scale, acc);
                accmin = fmaf((float)mq[q], dscale, accmin);
            }
        }
    }
    return acc - accmin;
}

/* amd-nv-cpu.ll:1836-2031 with build.rs:871-884: Q6_K under a 256 step. Chain
 * l (0..7) takes, from every 32-value group, the scaled dot of its four-value
 * word l (slice 2k + l/4, word l%4), less 32 times the scaled code sums of
 * group l; each chain meets its own fma once per block; a fixed tree adds the
 * eight chains. */
static float row_q6k_256(const uint8_t* row, int64_t cols, const float* rd, const int8_t* rc) {
    float f[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t b = 0; b < cols / 256; ++b) {
        const uint8_t* blk = row + b * 210;
        const int8_t* c = rc + b * 256;
        int32_t ints[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int s = 0; s < 16; ++s) {
            const int scale = (int8_t)blk[192 + s];
            for (int w = 0; w < 4; ++w) {
                int32_t dot = 0, sum = 0;
                for (int i = 0; i < 4; ++i) {
                    const int n = s * 16 + w * 4 + i;
                    dot += q6k_code(blk, n) * c[n];
                    sum += c[n];
                }
                ints[(s & 1) * 4 + w] += scale * dot;
                ints[s >> 1] += -32 * (scale * sum);
            }
        }
        const float scale = rd[b * 8] * f16_at(blk + 208);
        for (int l = 0; l < 8; ++l) f[l] = fmaf(scale, (float)ints[l], f[l]);
    }
    const float t0 = f[0] + f[4], t1 = f[1] + f[5], t2 = f[2] + f[6], t3 = f[3] + f[7];
    const float u0 = t0 + t2, u1 = t1 + t3;
    return u0 + u1;
}

int orc_int8_matvec(int format, const uint8_t* bytes, int64_t rows, int64_t cols, const float* x, int m_count,
                    int step, int tail, float* y) {
    if (format != 2 && format != 8 && format != 12 && format != 14) return -1;
    if (!shape_ok(format, rows, cols) || m_count < 1 || (step != 32 && step != 256)) return -1;
    const int64_t rbytes = row_bytes_of(format, cols);
    float* rd = (float*)malloc((size_t)(cols / 32) * sizeof(float));
    int8_t* rc = (int8_t*)malloc((size_t)cols);
    if (!rd || !rc) {
        free(rd);
        free(rc);
        return -2;
    }
    for (int m = 0; m < m_count; ++m) {
        orc_q8_records(x + (int64_t)m * cols, cols, step, rd, rc);
        const int whole = m >= m_count - m_count % 4 || (tail && m == m_count - 1);
        for (int64_t n = 0; n < rows; ++n) {
            const uint8_t* row = bytes + n * rbytes;
            float v;
            if (step == 256 && format == 12)
                v = row_q4k_256(row, cols, rd, rc, whole);
            else if (step == 256 && format == 14)
                v = row_q6k_256(row, cols, rd, rc);
            else
                v = row_slices(format, row, cols, rd, rc);
            y[(int64_t)m * rows + n] = v;
        }
    }
    free(rd);
    free(rc);
    return 0;
}

/* IEEE binary16 encode with round half to even, subnormals and overflow to
 * infinity (what LLVM's fptrunc float -> half does on recipe's device). */
uint16_t orc_fp16_rne(float value) {
    uint32_t x;
    memcpy(&x, &value, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t a = x & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0u));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 */
    if (a < 0x38800000u) {                                   /* below 2^-14 */
        const int e = (int)(a >> 23);
        if (e < 102) return sign;
        const uint32_t m = (a & 0x7fffffu) | 0x800000u;
        const int shift = 126 - e;
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t q = (a >> 13) - (112u << 10);
    const uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
}

/* recipe.rs:8016-8080 (emit_requantize, DeviceQuantizer::Q8_0) over the
 * decoded weight, 32 values at a time. */
int orc_requantize_q8_0(int format, const uint8_t* bytes, int64_t rows, int64_t cols, uint8_t* out) {
    if (format != 1 && format != 2 && format != 8 && format != 14) return -1;
    if (!shape_ok(format, rows, cols) || cols % 32 != 0) return -1;
    const int bv = orc_block_values(format), bb = orc_block_bytes(format);
    const int64_t rbytes = row_bytes_of(format, cols);
    for (int64_t r = 0; r < rows; ++r) {
        const uint8_t* row = bytes + r * rbytes;
        for (int64_t b = 0; b < cols / 32; ++b) {
            float v[32];
            for (int i = 0; i < 32; ++i) {
                const int64_t k = b * 32 + i;
                v[i] = (float)orc_dequant_value(format, row + (k / bv) * bb, (int)(k % bv));
            }
            float e = 0.0f;
            for (int i = 0; i < 32; ++i)
                if (fabsf(v[i]) > fabsf(e)) e = v[i];
            const float scale = fabsf(e) / 127.0f;
            const float inverse = scale == 0.0f ? 0.0f : 1.0f / scale;
            uint8_t* blk = out + (r * (cols / 32) + b) * 34;
            const uint16_t d = orc_fp16_rne(scale);
            blk[0] = (uint8_t)(d & 0xff);
            blk[1] = (uint8_t)(d >> 8);
            for (int i = 0; i < 32; ++i) {
                const float q = v[i] * inverse;
                const float rounded = q >= 0.0f ? q + 0.5f : q + -0.5f;
                int c = (int)rounded; /* toward zero */
                if (c < -128) c = -128;
                if (c > 127) c = 127;
                blk[2 + i] = (uint8_t)(int8_t)c;
            }
        }
    }
    return 0;
}
