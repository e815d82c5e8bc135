/*
 * recipe's CPU float path for the GGUF matvec, written for speed: the timed
 * CPU baseline of bench.py. TEST INFRASTRUCTURE (never part of the product).
 *
 * Same arithmetic as orc_matvec_recipe_f32 in oracle.c, value for value: each
 * weight is the f64 decode of its block rounded to fp32 (recipe's state-type
 * decode, recipe.rs:3687-3833), a run of `dot_run` values is an fp32 fma
 * chain from zero in index order (emit_run_decoder, recipe.rs:7826-7919), and
 * the runs of a row are added in order into its fp32 sum (packed_lanes_body,
 * amd-nv-cpu.ll:3053-3088). What differs is only the schedule recipe's
 * compiled path also uses: the block header (scales, minimums) is decoded
 * once per block instead of once per value, and eight rows run side by side,
 * one per SIMD lane (packed_lanes, amd-nv-cpu.ll:2304-3508), each lane
 * keeping its own row's sequential chain. tests/test_oracle.py checks the
 * outputs bit for bit against orc_matvec_recipe_f32.
 */
#include "oracle.h"

#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define LANES 8

static double half_value(const uint8_t* b) { return (double)orc_f32_from_fp16((uint16_t)(b[0] | (b[1] << 8))); }

/* One block of one row, decoded into w[j * LANES + lane], j < block values. */
static void decode_block(int format, const uint8_t* b, float* w, int lane) {
    switch (format) {
        case ORC_Q8_0: {
            const double d = half_value(b);
            for (int j = 0; j < 32; ++j) w[j * LANES + lane] = (float)((double)(int8_t)b[2 + j] * d);
            break;
        }
        case ORC_Q4_0: {
            const double d = half_value(b);
            for (int j = 0; j < 16; ++j) {
                w[j * LANES + lane] = (float)((double)((int)(b[2 + j] & 15) - 8) * d);
                w[(j + 16) * LANES + lane] = (float)((double)((int)(b[2 + j] >> 4) - 8) * d);
            }
            break;
        }
        case ORC_Q4_K: {
            const double d = half_value(b), dmin = half_value(b + 2);
            for (int sub = 0; sub < 8; ++sub) {
                int sc, mn;
                if (sub < 4) {
                    sc = b[4 + sub] & 63;
                    mn = b[8 + sub] & 63;
                } else {
                    sc = (b[8 + sub] & 15) | ((b[sub] >> 6) << 4);
                    mn = (b[8 + sub] >> 4) | ((b[4 + sub] >> 6) << 4);
                }
                const double step = d * (double)sc, base = dmin * (double)mn;
                const uint8_t* q = b + 16 + (sub / 2) * 32;
                const int shift = (sub % 2) * 4;
                for (int j = 0; j < 32; ++j)
                    w[(sub * 32 + j) * LANES + lane] = (float)(step * (double)((q[j] >> shift) & 15) - base);
            }
            break;
        }
        case ORC_Q6_K: {
            const double d = half_value(b + 208);
            for (int chunk = 0; chunk < 2; ++chunk)
                for (int group = 0; group < 4; ++group)
                    for (int half = 0; half < 2; ++half) {
                        const double scaled = d * (double)(int8_t)b[192 + chunk * 8 + group * 2 + half];
                        for (int k = 0; k < 16; ++k) {
                            const int within = half * 16 + k;
                            const int low = b[chunk * 64 + within + 32 * (group & 1)];
                            const int high = b[chunk * 32 + within + 128];
                            const int code = (((low >> (4 * (group / 2))) & 15) | (((high >> (2 * group)) & 3) << 4)) - 32;
                            w[(chunk * 128 + group * 32 + within) * LANES + lane] = (float)(scaled * (double)code);
                        }
                    }
            break;
        }
        default: break;
    }
}

typedef struct {
    int format;
    const uint8_t* bytes;
    int64_t rows, cols, row_begin, row_end;
    const float* x;
    int m_count;
    int64_t ldx, ldy;
    float* y;
} fast_job;

static void* fast_rows(void* arg) {
    const fast_job* job = (const fast_job*)arg;
    const int format = job->format;
    const int bv = orc_block_values(format), bb = orc_block_bytes(format);
    const int64_t nb = job->cols / bv;
    /* a run is the whole block here: 32 values for Q4_0 / Q8_0, 256 for the K formats */
    float* w = (float*)aligned_alloc(64, sizeof(float) * (size_t)bv * LANES);
    float* total = (float*)malloc(sizeof(float) * (size_t)job->m_count * LANES);
    for (int64_t r0 = job->row_begin; r0 < job->row_end; r0 += LANES) {
        const int lanes = job->row_end - r0 < LANES ? (int)(job->row_end - r0) : LANES;
        memset(total, 0, sizeof(float) * (size_t)job->m_count * LANES);
        memset(w, 0, sizeof(float) * (size_t)bv * LANES);
        for (int64_t blk = 0; blk < nb; ++blk) {
            for (int l = 0; l < lanes; ++l) decode_block(format, job->bytes + ((r0 + l) * nb + blk) * bb, w, l);
            for (int m = 0; m < job->m_count; ++m) {
                const float* xm = job->x + (int64_t)m * job->ldx + blk * bv;
                float part[LANES] = {0};
                for (int j = 0; j < bv; ++j) {
                    const float xj = xm[j];
                    for (int l = 0; l < LANES; ++l) part[l] = __builtin_fmaf(w[j * LANES + l], xj, part[l]);
                }
                for (int l = 0; l < LANES; ++l) total[m * LANES + l] = total[m * LANES + l] + part[l];
            }
        }
        for (int m = 0; m < job->m_count; ++m)
            for (int l = 0; l < lanes; ++l) job->y[(int64_t)m * job->ldy + r0 + l] = total[m * LANES + l];
    }
    free(w);
    free(total);
    return NULL;
}

int orc_matvec_recipe_fast(int format, const uint8_t* bytes, int64_t rows, int64_t cols, const float* x, int m_count,
                           int64_t ldx, float* y, int64_t ldy, int threads) {
    const int bv = orc_block_values(format);
    if (format != ORC_Q4_0 && format != ORC_Q8_0 && format != ORC_Q4_K && format != ORC_Q6_K) return -1;
    if (rows < 0 || cols <= 0 || cols % bv != 0 || m_count <= 0) return -1;
    const int64_t groups = (rows + LANES - 1) / LANES;
    if (threads < 1) threads = 1;
    if (threads > groups) threads = groups > 0 ? (int)groups : 1;
    pthread_t* tids = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    fast_job* jobs = (fast_job*)malloc(sizeof(fast_job) * (size_t)threads);
    for (int t = 0; t < threads; ++t) {
        const int64_t g0 = groups * t / threads, g1 = groups * (t + 1) / threads;
        const int64_t begin = g0 * LANES, end = g1 * LANES < rows ? g1 * LANES : rows;
        fast_job job = {format, bytes, rows, cols, begin, end, x, m_count, ldx, ldy, y};
        jobs[t] = job;
    }
    if (threads == 1) {
        fast_rows(&jobs[0]);
    } else {
        for (int t = 0; t < threads; ++t) pthread_create(&tids[t], NULL, fast_rows, &jobs[t]);
        for (int t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
    }
    free(tids);
    free(jobs);
    return 0;
}
