/*
 * barq_oracle.c — CPU restatement of barq-inference's quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY (see barq_oracle.h).  Compiled with
 * -ffp-contract=off so every f32 product and sum rounds separately, as the
 * reference's Rust does.  Citations are /root/reference paths.
 */
#include "barq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* small helpers                                                             */
/* ------------------------------------------------------------------------ */

#define FLT_EPSILON_ORC 1.1920929e-7f   /* f32::EPSILON = 2^-23 */

static float f32_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits_from_f32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static uint16_t rd_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static float rd_f32(const uint8_t* p) {
    uint32_t u = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
    return f32_from_bits(u);
}
static void wr_u16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }
static void wr_f32(uint8_t* p, float f) {
    uint32_t u = bits_from_f32(f);
    p[0] = (uint8_t)u; p[1] = (uint8_t)(u >> 8); p[2] = (uint8_t)(u >> 16); p[3] = (uint8_t)(u >> 24);
}

size_t orc_block_elems(int type) {
    switch (type) {
    case ORC_F32: case ORC_F16: return 1;
    case ORC_Q4_0: case ORC_Q8_0: case ORC_Q4_0_BARQ: return 32;   /* gguf.rs:170-172 */
    case ORC_Q4_K: case ORC_Q6_K: case ORC_Q8_K: return 256;       /* gguf.rs:173-182 */
    default: return 0;
    }
}

size_t orc_block_bytes(int type) {
    switch (type) {
    case ORC_F32: return 4;
    case ORC_F16: return 2;
    case ORC_Q4_0: return 18;        /* llama.cpp block_q4_0 */
    case ORC_Q4_0_BARQ: return 20;   /* gguf.rs:529-530 */
    case ORC_Q8_0: return 34;        /* gguf.rs:645 */
    case ORC_Q4_K: return 144;       /* gguf.rs:747 */
    case ORC_Q6_K: return 210;       /* gguf.rs:854 */
    case ORC_Q8_K: return 292;       /* llama.cpp block_q8_K: f32 d, i8 qs[256], i16 bsums[16] */
    default: return 0;
    }
}

/* half 2.7.1 f16::to_f32: exact IEEE widening; NaNs keep their payload with
   the quiet bit set (the crate's fallback and F16C both do). */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    if (exp == 0) {
        if (man == 0) return f32_from_bits(sign);
        /* subnormal: value = man * 2^-24, renormalise */
        int e = 0;
        while (!(man & 0x400u)) { man <<= 1; e++; }
        man &= 0x3FFu;
        return f32_from_bits(sign | ((uint32_t)(127 - 15 + 1 - e) << 23) | (man << 13));
    }
    if (exp == 31) {
        if (man == 0) return f32_from_bits(sign | 0x7F800000u);
        return f32_from_bits(sign | 0x7FC00000u | (man << 13));
    }
    return f32_from_bits(sign | ((exp + 112u) << 23) | (man << 13));
}

/* binary32 -> binary16, round to nearest, ties to even. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x = bits_from_f32(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFF) {
        if (man == 0) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7E00u | (man >> 13));
    }
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);           /* overflow -> inf */
    if (e <= 0) {                                              /* subnormal or zero */
        if (e < -10) return sign;                              /* < half of min subnormal */
        uint32_t m = man | 0x800000u;                          /* 24-bit significand */
        int shift = 14 - e;                                    /* 24 -> (11+e-1) bits */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;  /* carry may reach inf: correct */
    return (uint16_t)(sign | q);
}

/* ------------------------------------------------------------------------ */
/* block decoders                                                            */
/* ------------------------------------------------------------------------ */

/* barq_core/src/gguf.rs:521-578 (load_q4_0), identical to
   quant/src/q4_0.rs:69-115: f32 LE scale + 16 bytes; element i is nibble
   (i%2 ? high : low) of byte i/2, sign-extended (q>=8 -> q-16),
   value = q as f32 * scale. */
size_t orc_dequant_q4_0_barq(const uint8_t* data, size_t total_elements, float* out) {
    size_t n_blocks = (total_elements + 31) / 32;
    size_t w = 0;
    for (size_t b = 0; b < n_blocks; b++) {
        const uint8_t* blk = data + b * 20;
        float scale = rd_f32(blk);
        const uint8_t* quants = blk + 4;
        for (int i = 0; i < 32 && w < total_elements; i++) {
            int shift = (i % 2 == 0) ? 0 : 4;
            int q = (quants[i / 2] >> shift) & 0x0F;
            if (q >= 8) q -= 16;
            out[w++] = (float)q * scale;
        }
    }
    return w;
}

/* Byte adapter GGUF block_q4_0 (f16 d, element i<16 = low nibble of byte i,
   element i>=16 = high nibble of byte i-16, value (nib-8)*d) -> the
   reference's 20-B layout.  scale = f16->f32(d) is exact; the reference
   nibble for element i is gguf_nib(i) ^ 8, which sign-extends to nib-8. */
void orc_q4_0_gguf_to_barq(const uint8_t* gguf, size_t n_blocks, uint8_t* barq) {
    for (size_t b = 0; b < n_blocks; b++) {
        const uint8_t* s = gguf + b * 18;
        uint8_t* d = barq + b * 20;
        wr_f32(d, orc_f16_to_f32(rd_u16(s)));
        memset(d + 4, 0, 16);
        for (int i = 0; i < 32; i++) {
            int nib = (i < 16) ? (s[2 + i] & 0x0F) : (s[2 + i - 16] >> 4);
            int rn = (nib ^ 8) & 0x0F;
            d[4 + i / 2] |= (uint8_t)(rn << ((i % 2) ? 4 : 0));
        }
    }
}

size_t orc_dequant_q4_0_gguf(const uint8_t* data, size_t total_elements, float* out) {
    size_t n_blocks = (total_elements + 31) / 32;
    uint8_t tmp[20];
    size_t w = 0;
    for (size_t b = 0; b < n_blocks; b++) {
        float blk[32];
        orc_q4_0_gguf_to_barq(data + b * 18, 1, tmp);
        orc_dequant_q4_0_barq(tmp, 32, blk);
        for (int i = 0; i < 32 && w < total_elements; i++) out[w++] = blk[i];
    }
    return w;
}

/* gguf.rs:634-681 (load_q8_0): f16 d + 32 bytes; value = (q as i8) as f32 * d */
size_t orc_dequant_q8_0(const uint8_t* data, size_t total_elements, float* out) {
    size_t n_blocks = (total_elements + 31) / 32;
    size_t w = 0;
    for (size_t b = 0; b < n_blocks; b++) {
        const uint8_t* blk = data + b * 34;
        float scale = orc_f16_to_f32(rd_u16(blk));
        for (int i = 0; i < 32 && w < total_elements; i++) out[w++] = (float)(int8_t)blk[2 + i] * scale;
    }
    return w;
}

/* gguf.rs:825-837 (get_scale_min_k4) */
void orc_get_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* quant/src/q5_k.rs:175-182: the encoder of the same 12-byte packing. */
void orc_pack_scale_min_k4(const uint8_t ls[8], const uint8_t lm[8], uint8_t out[12]) {
    memset(out, 0, 12);
    for (int j = 0; j < 8; j++) {
        if (j < 4) {
            out[j] = ls[j];
            out[j + 4] = lm[j];
        } else {
            out[j + 4] = (uint8_t)((ls[j] & 0x0f) | ((lm[j] & 0x0f) << 4));
            out[j - 4] |= (uint8_t)((ls[j] >> 4) << 6);
            out[j] |= (uint8_t)((lm[j] >> 4) << 6);
        }
    }
}

/* gguf.rs:730-823 (load_q4_k): d, dmin (f16), scales[12], qs[128].
   For each 64-chunk j: (sc,m)=gsm(is); d1=d*sc; m1=dmin*m; 32 x
   (d1*(qs&15) - m1); then gsm(is+1) with qs>>4; is += 2.  Products and the
   difference round separately (no FMA), gguf.rs:804,814. */
size_t orc_dequant_q4_k(const uint8_t* data, size_t total_elements, float* out) {
    size_t n_blocks = (total_elements + 255) / 256;
    size_t w = 0;
    for (size_t b = 0; b < n_blocks; b++) {
        const uint8_t* blk = data + b * 144;
        float d = orc_f16_to_f32(rd_u16(blk));
        float dmin = orc_f16_to_f32(rd_u16(blk + 2));
        const uint8_t* scales = blk + 4;
        const uint8_t* qs = blk + 16;
        int is = 0;
        for (int j = 0; j < 256; j += 64) {
            uint8_t sc, m;
            orc_get_scale_min_k4(is, scales, &sc, &m);
            float d1 = d * (float)sc;
            float min1 = dmin * (float)m;
            for (int l = 0; l < 32; l++) {
                float p = d1 * (float)(qs[j / 2 + l] & 0x0F);
                if (w < total_elements) out[w] = p - min1;
                w++;
            }
            orc_get_scale_min_k4(is + 1, scales, &sc, &m);
            float d2 = d * (float)sc;
            float min2 = dmin * (float)m;
            for (int l = 0; l < 32; l++) {
                float p = d2 * (float)(qs[j / 2 + l] >> 4);
                if (w < total_elements) out[w] = p - min2;
                w++;
            }
            is += 2;
        }
    }
    return w < total_elements ? w : total_elements;
}

/* gguf.rs:839-914 (load_q6_k): ql[128], qh[64], i8 scales[16], f16 d. */
size_t orc_dequant_q6_k(const uint8_t* data, size_t total_elements, float* out) {
    size_t n_blocks = (total_elements + 255) / 256;
    for (size_t b = 0; b < n_blocks; b++) {
        const uint8_t* ql = data + b * 210;
        const uint8_t* qh = ql + 128;
        const uint8_t* sc = ql + 192;
        float d = orc_f16_to_f32(rd_u16(ql + 208));
        float tmp[256];
        for (int n = 0; n < 256; n += 128) {
            int off_ql = n / 2, off_qh = n / 4, off_sc = n / 16;
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                float d0 = d * (float)(int8_t)sc[off_sc + is + 0];
                float d1 = d * (float)(int8_t)sc[off_sc + is + 2];
                float d2 = d * (float)(int8_t)sc[off_sc + is + 4];
                float d3 = d * (float)(int8_t)sc[off_sc + is + 6];
                uint8_t h = qh[off_qh + l];
                int v0 = (int)(int8_t)((ql[off_ql + l] & 0xF) | (((h >> 0) & 3) << 4)) - 32;
                int v1 = (int)(int8_t)((ql[off_ql + l + 32] & 0xF) | (((h >> 2) & 3) << 4)) - 32;
                int v2 = (int)(int8_t)((ql[off_ql + l] >> 4) | (((h >> 4) & 3) << 4)) - 32;
                int v3 = (int)(int8_t)((ql[off_ql + l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32;
                tmp[n + l + 0] = d0 * (float)v0;
                tmp[n + l + 32] = d1 * (float)v1;
                tmp[n + l + 64] = d2 * (float)v2;
                tmp[n + l + 96] = d3 * (float)v3;
            }
        }
        size_t base = b * 256;
        for (int i = 0; i < 256 && base + i < total_elements; i++) out[base + i] = tmp[i];
    }
    return total_elements;
}

/* llama.cpp dequantize_row_q8_K: y = d * q */
size_t orc_dequant_q8_k(const uint8_t* data, size_t total_elements, float* out) {
    size_t n_blocks = (total_elements + 255) / 256;
    size_t w = 0;
    for (size_t b = 0; b < n_blocks; b++) {
        const uint8_t* blk = data + b * 292;
        float d = rd_f32(blk);
        for (int i = 0; i < 256 && w < total_elements; i++) out[w++] = d * (float)(int8_t)blk[4 + i];
    }
    return w;
}

size_t orc_dequantize(int type, const uint8_t* data, size_t total_elements, float* out) {
    switch (type) {
    case ORC_F32:
        memcpy(out, data, total_elements * 4);
        return total_elements;
    case ORC_F16:  /* gguf.rs:456-469 */
        for (size_t i = 0; i < total_elements; i++) out[i] = orc_f16_to_f32(rd_u16(data + 2 * i));
        return total_elements;
    case ORC_Q4_0: return orc_dequant_q4_0_gguf(data, total_elements, out);
    case ORC_Q4_0_BARQ: return orc_dequant_q4_0_barq(data, total_elements, out);
    case ORC_Q8_0: return orc_dequant_q8_0(data, total_elements, out);
    case ORC_Q4_K: return orc_dequant_q4_k(data, total_elements, out);
    case ORC_Q6_K: return orc_dequant_q6_k(data, total_elements, out);
    case ORC_Q8_K: return orc_dequant_q8_k(data, total_elements, out);
    default: return (size_t)-1;
    }
}

/* ------------------------------------------------------------------------ */
/* activation quantizers — the reference has none (Q8_K is an enum id only, */
/* gguf.rs:132, quant.rs:29); these follow llama.cpp's public                */
/* quantize_row_q8_0_ref / quantize_row_q8_K_ref.                           */
/* ------------------------------------------------------------------------ */

void orc_quantize_q8_0(const float* x, size_t k, uint8_t* out) {
    size_t nb = k / 32;
    for (size_t b = 0; b < nb; b++) {
        const float* xb = x + b * 32;
        uint8_t* y = out + b * 34;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) {
            float v = fabsf(xb[j]);
            amax = amax > v ? amax : v;
        }
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        wr_u16(y, orc_f32_to_f16(d));
        for (int j = 0; j < 32; j++) {
            float x0 = xb[j] * id;
            y[2 + j] = (uint8_t)(int8_t)roundf(x0);   /* half away from zero */
        }
    }
}

void orc_quantize_q8_k(const float* x, size_t k, uint8_t* out) {
    size_t nb = k / 256;
    for (size_t b = 0; b < nb; b++) {
        const float* xb = x + b * 256;
        uint8_t* y = out + b * 292;
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < 256; j++) {
            float ax = fabsf(xb[j]);
            if (ax > amax) { amax = ax; max = xb[j]; }
        }
        if (amax == 0.0f) {
            memset(y, 0, 292);   /* d = 0, qs = 0, bsums = 0 */
            continue;
        }
        float iscale = -127.0f / max;
        int8_t q[256];
        for (int j = 0; j < 256; j++) {
            int v = (int)rintf(iscale * xb[j]);   /* round to nearest, ties to even */
            q[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int j = 0; j < 256; j++) y[4 + j] = (uint8_t)q[j];
        for (int g = 0; g < 16; g++) {
            int s = 0;
            for (int i = 0; i < 16; i++) s += q[16 * g + i];
            wr_u16(y + 260 + 2 * g, (uint16_t)(int16_t)s);
        }
        wr_f32(y, 1.0f / iscale);
    }
}

/* ------------------------------------------------------------------------ */
/* the reference's f32 GEMV / GEMM                                           */
/* ------------------------------------------------------------------------ */

/* LlamaTransformer::rms_norm (models/src/transformer.rs:148-172), row by
   row: eps' = eps.max(f32::EPSILON) (:158); sum_sq sequential over the row
   (:162, Iterator::sum folds left); mean_square = sum_sq / n (:163);
   rms_inv = 1.0 / (mean_square + eps').sqrt() (:164);
   y = hidden * rms_inv * weight, left to right (:166). */
void orc_rms_norm(const float* x, const float* w, size_t rows, size_t n, float eps, float* y) {
    const float e = eps > FLT_EPSILON_ORC ? eps : FLT_EPSILON_ORC;
    for (size_t r = 0; r < rows; r++) {
        const float* xr = x + r * n;
        float sum_sq = 0.0f;
        for (size_t j = 0; j < n; j++) {
            const float sq = xr[j] * xr[j];
            sum_sq = sum_sq + sq;
        }
        const float mean_square = sum_sq / (float)n;
        const float rms_inv = 1.0f / sqrtf(mean_square + e);
        for (size_t j = 0; j < n; j++) {
            const float t = xr[j] * rms_inv;
            y[r * n + j] = t * w[j];
        }
    }
}

void orc_gemv_f32(const float* a, const float* x, size_t m, size_t n, float* y) {
    for (size_t i = 0; i < m; i++) {
        float sum = 0.0f;
        for (size_t j = 0; j < n; j++) sum += a[i * n + j] * x[j];
        y[i] = sum;
    }
}

void orc_gemm_f32(const float* a, const float* b, size_t m, size_t k, size_t n, float* c) {
    for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < n; j++) {
            float sum = 0.0f;
            for (size_t kk = 0; kk < k; kk++) sum += a[i * k + kk] * b[kk * n + j];
            c[i * n + j] = sum;
        }
}

static int act_dequant(int act_type, const void* x, size_t k, float* out) {
    if (act_type == ORC_F32) { memcpy(out, x, k * sizeof(float)); return 0; }
    if (act_type == ORC_Q8_0 && k % 32 == 0) { orc_dequant_q8_0((const uint8_t*)x, k, out); return 0; }
    if (act_type == ORC_Q8_K && k % 256 == 0) { orc_dequant_q8_k((const uint8_t*)x, k, out); return 0; }
    return -1;
}

static size_t act_row_bytes(int act_type, size_t k) {
    if (act_type == ORC_F32) return k * 4;
    return k / orc_block_elems(act_type) * orc_block_bytes(act_type);
}

int orc_matmul(int w_type, const uint8_t* w, size_t n_rows, size_t k,
               int act_type, const void* x, size_t m, float* y) {
    size_t be = orc_block_elems(w_type), bb = orc_block_bytes(w_type);
    if (!be || !bb || w_type == ORC_Q8_K || k % be) return -1;
    if (act_type != ORC_F32 && act_type != ORC_Q8_0 && act_type != ORC_Q8_K) return -1;
    size_t row_bytes = k / be * bb;
    size_t xrb = act_row_bytes(act_type, k);
    float* xf = (float*)malloc(m * k * sizeof(float));
    float* wr = (float*)malloc(k * sizeof(float));
    if (!xf || !wr) { free(xf); free(wr); return -1; }
    for (size_t r = 0; r < m; r++)
        if (act_dequant(act_type, (const uint8_t*)x + r * xrb, k, xf + r * k)) { free(xf); free(wr); return -1; }
    for (size_t n = 0; n < n_rows; n++) {
        orc_dequantize(w_type, w + n * row_bytes, k, wr);
        for (size_t r = 0; r < m; r++) {
            const float* xr = xf + r * k;
            float sum = 0.0f;
            for (size_t kk = 0; kk < k; kk++) sum += xr[kk] * wr[kk];
            y[r * n_rows + n] = sum;
        }
    }
    free(xf); free(wr);
    return 0;
}

int orc_matvec(int w_type, const uint8_t* w, size_t n_rows, size_t k,
               int act_type, const void* x, float* y) {
    return orc_matmul(w_type, w, n_rows, k, act_type, x, 1, y);
}

/* ------------------------------------------------------------------------ */
/* quant crate / split-scale operator API                                    */
/* ------------------------------------------------------------------------ */

/* quant/src/q4_0.rs:23-67.  scale = max_abs/8 (0 if all zero);
   q = clamp((x/scale).round() as i8, -8, 7) — Rust's round is half away
   from zero and `as i8` saturates. */
size_t orc_q4_0_quantize_barq(const float* x, size_t n, uint8_t* out) {
    size_t n_blocks = (n + 31) / 32;
    size_t o = 0;
    for (size_t b = 0; b < n_blocks; b++) {
        size_t start = b * 32, end = start + 32 < n ? start + 32 : n;
        float max_abs = 0.0f;
        for (size_t i = start; i < end; i++) { float a = fabsf(x[i]); max_abs = max_abs > a ? max_abs : a; }
        float scale = max_abs == 0.0f ? 0.0f : max_abs / 8.0f;
        size_t qlen = (end - start + 1) / 2;
        uint8_t quants[16];
        memset(quants, 0, sizeof quants);
        for (size_t i = start; i < end; i++) {
            int q;
            if (scale == 0.0f) q = 0;
            else {
                float r = roundf(x[i] / scale);
                if (r != r) q = 0;                       /* NaN as i8 -> 0 */
                else if (r > 127.0f) q = 127;
                else if (r < -128.0f) q = -128;
                else q = (int)r;
            }
            if (q < -8) q = -8;
            if (q > 7) q = 7;
            size_t rel = i - start;
            quants[rel / 2] |= (uint8_t)(((uint8_t)q & 0x0F) << ((rel % 2) ? 4 : 0));
        }
        wr_f32(out + o, scale);
        memcpy(out + o + 4, quants, qlen);
        o += 4 + qlen;
    }
    return o;
}

/* cuda_quant.rs:44-75 */
void orc_dequantize_packed_4bit_split(const uint8_t* quants, size_t n_quants,
                                      const float* scales, size_t n_scales,
                                      size_t block_size, float* out, size_t n_out) {
    size_t q_offset = 0;
    for (size_t b = 0; b < n_scales; b++) {
        size_t start = b * block_size;
        if (start >= n_out) break;
        size_t end = start + block_size < n_out ? start + block_size : n_out;
        float scale = scales[b];
        for (size_t i = start; i < end; i++) {
            size_t rel = i - start;
            size_t byte_idx = rel / 2;
            int shift = (rel % 2 == 0) ? 0 : 4;
            if (q_offset + byte_idx < n_quants) {
                int q = (quants[q_offset + byte_idx] >> shift) & 0x0F;
                if (q >= 8) q -= 16;
                out[i] = (float)q * scale;
            }
        }
        q_offset += (block_size + 1) / 2;
    }
}

/* cuda_quant.rs:77-102 */
void orc_dequantize_signed_8bit_split(const uint8_t* quants, size_t n_quants,
                                      const float* scales, size_t n_scales,
                                      size_t block_size, float* out, size_t n_out) {
    for (size_t b = 0; b < n_scales; b++) {
        size_t start = b * block_size;
        if (start >= n_out) break;
        size_t end = start + block_size < n_out ? start + block_size : n_out;
        size_t q_offset = b * block_size;
        for (size_t i = start; i < end; i++) {
            size_t rel = i - start;
            if (q_offset + rel < n_quants) out[i] = (float)(int8_t)quants[q_offset + rel] * scales[b];
        }
    }
}

/* cuda_quant.rs:104-126: b_dequant is zero-initialised (k*n), filled by the
   split decoder, then blas::gemm_f32(a, b, m, k, n). */
void orc_quantized_matmul_split(const float* a, const uint8_t* bq, size_t n_bq,
                                const float* bscales, size_t n_bscales,
                                size_t m, size_t n, size_t k, int quant_is_q8_0,
                                size_t block_size, float* c) {
    float* b = (float*)calloc(k * n, sizeof(float));
    if (!b) return;
    if (quant_is_q8_0) orc_dequantize_signed_8bit_split(bq, n_bq, bscales, n_bscales, block_size, b, k * n);
    else orc_dequantize_packed_4bit_split(bq, n_bq, bscales, n_bscales, block_size, b, k * n);
    orc_gemm_f32(a, b, m, k, n, c);
    free(b);
}

/* ------------------------------------------------------------------------ */
/* fused MoE helpers (models/src/moe_fused.rs)                               */
/* ------------------------------------------------------------------------ */

size_t orc_moe_select_top_k(const float* logits, size_t rows, size_t cols,
                            size_t k, int32_t* ids, float* weights) {
    if (cols == 0) return 0;                                   /* :115-119 */
    size_t kk = k < 1 ? 1 : (k > cols ? cols : k);             /* :121 */
    int32_t* order = (int32_t*)malloc(cols * sizeof(int32_t));
    float* ex = (float*)malloc(kk * sizeof(float));
    if (!order || !ex) { free(order); free(ex); return 0; }
    for (size_t r = 0; r < rows; r++) {
        const float* row = logits + r * cols;
        /* stable sort by value, descending (Rust sort_by is stable; NaN
           compares Equal via unwrap_or) — :124-126 */
        for (size_t i = 0; i < cols; i++) order[i] = (int32_t)i;
        for (size_t i = 1; i < cols; i++) {
            int32_t cur = order[i];
            size_t j = i;
            while (j > 0 && row[order[j - 1]] < row[cur]) { order[j] = order[j - 1]; j--; }
            order[j] = cur;
        }
        float mx = -INFINITY;                                  /* :129-132 */
        for (size_t i = 0; i < kk; i++) mx = fmaxf(mx, row[order[i]]);
        float denom = 0.0f;                                    /* :133-137 */
        for (size_t i = 0; i < kk; i++) { ex[i] = expf(row[order[i]] - mx); denom += ex[i]; }
        if (denom < 1.1920929e-7f) denom = 1.1920929e-7f;      /* .max(f32::EPSILON) */
        for (size_t i = 0; i < kk; i++) {
            ids[r * kk + i] = order[i];
            weights[r * kk + i] = ex[i] / denom;
        }
    }
    free(order); free(ex);
    return kk;
}

void orc_moe_reduce_experts(const int32_t* ids, const float* weights, size_t rows, size_t k,
                            size_t max_active, float min_weight, int32_t* out_ids, float* out_weights) {
    /* reduce_expert_assignments (moe_fused.rs:147-194).  A row's assignments
       are its k slots; a slot with id < 0 is absent (an assignment dropped
       earlier).  Output: the kept assignments first, then id -1 / weight 0. */
    const size_t keep_max = max_active > 0 ? max_active : 1;    /* .max(1), :180 */
    int32_t* ci = (int32_t*)malloc((k ? k : 1) * sizeof(int32_t));
    float* cw = (float*)malloc((k ? k : 1) * sizeof(float));
    if (!ci || !cw) { free(ci); free(cw); return; }
    for (size_t r = 0; r < rows; r++) {
        const int32_t* ri = ids + r * k;
        const float* rw = weights + r * k;
        size_t n = 0;
        for (size_t i = 0; i < k; i++)                          /* filter(weight >= min_weight), :161 */
            if (ri[i] >= 0 && rw[i] >= min_weight) { ci[n] = ri[i]; cw[n] = rw[i]; n++; }
        if (n == 0) {
            /* max_by with partial_cmp().unwrap_or(Equal) (:165-171): the running
               maximum is replaced unless it compares Greater, so among equal
               weights (and NaN) the later slot wins */
            long best = -1;
            for (size_t i = 0; i < k; i++) {
                if (ri[i] < 0) continue;
                if (best < 0 || !(rw[best] > rw[i])) best = (long)i;
            }
            if (best >= 0) { ci[0] = ri[best]; cw[0] = rw[best]; n = 1; }
        }
        /* stable sort by weight, descending (:177) */
        for (size_t i = 1; i < n; i++) {
            int32_t ti = ci[i]; float tw = cw[i];
            size_t j = i;
            while (j > 0 && cw[j - 1] < tw) { ci[j] = ci[j - 1]; cw[j] = cw[j - 1]; j--; }
            ci[j] = ti; cw[j] = tw;
        }
        if (n > keep_max) n = keep_max;                         /* truncate, :178 */
        float sum = -0.0f;                                      /* Sum<f32>: sequential fold, :180-184 */
        for (size_t i = 0; i < n; i++) sum += cw[i];
        sum = fmaxf(sum, 1.1920929e-7f);                        /* .max(f32::EPSILON) */
        for (size_t i = 0; i < k; i++) {
            out_ids[r * k + i] = i < n ? ci[i] : -1;
            out_weights[r * k + i] = i < n ? cw[i] / sum : 0.0f;
        }
    }
    free(ci); free(cw);
}

void orc_moe_batch_by_expert(const int32_t* ids, const float* weights,
                             size_t rows, size_t k, size_t n_experts,
                             int32_t* offsets, int32_t* tokens, float* wts) {
    /* :196-223 — tokens visited in ascending order, each token's ids in
       routing order; ids >= n_experts are skipped (batches.get_mut). */
    for (size_t e = 0; e <= n_experts; e++) offsets[e] = 0;
    for (size_t t = 0; t < rows; t++)
        for (size_t i = 0; i < k; i++) {
            int32_t e = ids[t * k + i];
            if (e >= 0 && (size_t)e < n_experts) offsets[e + 1]++;
        }
    for (size_t e = 0; e < n_experts; e++) offsets[e + 1] += offsets[e];
    int32_t* fill = (int32_t*)calloc(n_experts ? n_experts : 1, sizeof(int32_t));
    if (!fill) return;
    for (size_t t = 0; t < rows; t++)
        for (size_t i = 0; i < k; i++) {
            int32_t e = ids[t * k + i];
            if (e < 0 || (size_t)e >= n_experts) continue;
            int32_t pos = offsets[e] + fill[e]++;
            tokens[pos] = (int32_t)t;
            wts[pos] = weights[t * k + i];
        }
    free(fill);
}

int orc_moe_dispatch(const float* input, size_t rows, size_t hidden,
                     size_t n_experts, const int32_t* ids, const float* weights,
                     size_t k, orc_expert_fn fn, void* ctx, float* out) {
    if (n_experts == 0) return -1;                             /* :254-256 */
    size_t total = rows * k;
    int32_t* offsets = (int32_t*)malloc((n_experts + 1) * sizeof(int32_t));
    int32_t* tokens = (int32_t*)malloc((total ? total : 1) * sizeof(int32_t));
    float* wts = (float*)malloc((total ? total : 1) * sizeof(float));
    float* bin = (float*)malloc((total ? total : 1) * hidden * sizeof(float));
    float* bout = (float*)malloc((total ? total : 1) * hidden * sizeof(float));
    int rc = 0;
    if (!offsets || !tokens || !wts || !bin || !bout) { rc = -1; goto done; }
    memset(out, 0, rows * hidden * sizeof(float));             /* :260 */
    orc_moe_batch_by_expert(ids, weights, rows, k, n_experts, offsets, tokens, wts);
    for (size_t e = 0; e < n_experts; e++) {                   /* :263-300 */
        size_t b0 = (size_t)offsets[e], b1 = (size_t)offsets[e + 1];
        if (b0 == b1) continue;
        size_t nb = b1 - b0;
        for (size_t r = 0; r < nb; r++)
            memcpy(bin + r * hidden, input + (size_t)tokens[b0 + r] * hidden, hidden * sizeof(float));
        if (fn((int)e, bin, nb, hidden, bout, ctx)) { rc = -1; goto done; }
        for (size_t r = 0; r < nb; r++) {
            float w = wts[b0 + r];
            float* o = out + (size_t)tokens[b0 + r] * hidden;
            const float* s = bout + r * hidden;
            for (size_t h = 0; h < hidden; h++) o[h] += s[h] * w;
        }
    }
done:
    free(offsets); free(tokens); free(wts); free(bin); free(bout);
    return rc;
}

/* ---- dense FFN (models/src/transformer.rs:378-408) ------------------------ */

void orc_ffn_swiglu(const float* g, const float* u, size_t n, float* h) {
    /* :394-399 — (g * (1.0 / (1.0 + (-g).exp()))) * u, in this order */
    for (size_t i = 0; i < n; i++) {
        const float r = 1.0f / (1.0f + expf(-g[i]));
        const float a = g[i] * r;
        h[i] = a * u[i];
    }
}

static int q8_partner(int w_type) {
    return (w_type == ORC_Q4_K || w_type == ORC_Q6_K) ? ORC_Q8_K : ORC_Q8_0;
}

int orc_ffn(int gate_type, const uint8_t* gate, int up_type, const uint8_t* up,
            int down_type, const uint8_t* down, size_t n_embd, size_t n_ff,
            int act, const void* x, size_t m, float* out) {
    /* feed_forward: gate and up by proj_with_in_dim (:381-392, the matmul of
       :411-442), the SwiGLU, then down (:401-407) */
    const int lit = act == ORC_F32;
    const int pd = q8_partner(down_type);
    float* g = (float*)malloc(m * n_ff * sizeof(float));
    float* u = (float*)malloc(m * n_ff * sizeof(float));
    uint8_t* hq = NULL;
    int rc = -1;
    if (!g || !u) goto done;
    if (!lit && (act != q8_partner(gate_type) || act != q8_partner(up_type))) goto done;
    if (orc_matmul(gate_type, gate, n_ff, n_embd, act, x, m, g)) goto done;
    if (orc_matmul(up_type, up, n_ff, n_embd, act, x, m, u)) goto done;
    orc_ffn_swiglu(g, u, m * n_ff, g);
    if (lit) {
        rc = orc_matmul(down_type, down, n_embd, n_ff, ORC_F32, g, m, out);
    } else {
        const size_t rb = n_ff / orc_block_elems(pd) * orc_block_bytes(pd);
        if (n_ff % orc_block_elems(pd)) goto done;
        hq = (uint8_t*)malloc(m * rb);
        if (!hq) goto done;
        for (size_t r = 0; r < m; r++) {
            if (pd == ORC_Q8_K) orc_quantize_q8_k(g + r * n_ff, n_ff, hq + r * rb);
            else orc_quantize_q8_0(g + r * n_ff, n_ff, hq + r * rb);
        }
        rc = orc_matmul(down_type, down, n_embd, n_ff, pd, hq, m, out);
    }
done:
    free(g); free(u); free(hq);
    return rc;
}

struct moe_ffn_ctx {
    int gate_type, up_type, down_type, act;
    const uint8_t* const* gate;
    const uint8_t* const* up;
    const uint8_t* const* down;
    size_t n_ff;
};

/* One expert: fused_ffn (moe_fused.rs:84-92) = MatMul(silu(x G) * (x U), D)
   with Silu x/(1+exp(-x)) (ops.rs:191-211) and the elementwise a*b of
   fused_up_gate (:61-66).  With act == ORC_Q8_K the two contraction inputs
   are Q8_K-quantized first (the integer path the GPU runs). */
static int moe_expert_ffn(int e, const float* in, size_t rows, size_t hidden, float* out, void* vctx) {
    struct moe_ffn_ctx* c = (struct moe_ffn_ctx*)vctx;
    size_t n_ff = c->n_ff;
    float* g = (float*)malloc(rows * n_ff * sizeof(float));
    float* u = (float*)malloc(rows * n_ff * sizeof(float));
    uint8_t* qx = NULL;
    int rc = -1;
    if (!g || !u) goto done;
    if (c->act == ORC_Q8_K) {
        size_t qb = (n_ff > hidden ? n_ff : hidden) / 256 * 292;
        qx = (uint8_t*)malloc(rows * qb);
        if (!qx) goto done;
        for (size_t r = 0; r < rows; r++) orc_quantize_q8_k(in + r * hidden, hidden, qx + r * (hidden / 256 * 292));
        if (orc_matmul(c->gate_type, c->gate[e], n_ff, hidden, ORC_Q8_K, qx, rows, g)) goto done;
        if (orc_matmul(c->up_type, c->up[e], n_ff, hidden, ORC_Q8_K, qx, rows, u)) goto done;
    } else {
        if (orc_matmul(c->gate_type, c->gate[e], n_ff, hidden, ORC_F32, in, rows, g)) goto done;
        if (orc_matmul(c->up_type, c->up[e], n_ff, hidden, ORC_F32, in, rows, u)) goto done;
    }
    for (size_t i = 0; i < rows * n_ff; i++) {
        float a = g[i] / (1.0f + expf(-g[i]));
        g[i] = a * u[i];
    }
    if (c->act == ORC_Q8_K) {
        for (size_t r = 0; r < rows; r++) orc_quantize_q8_k(g + r * n_ff, n_ff, qx + r * (n_ff / 256 * 292));
        rc = orc_matmul(c->down_type, c->down[e], hidden, n_ff, ORC_Q8_K, qx, rows, out);
    } else {
        rc = orc_matmul(c->down_type, c->down[e], hidden, n_ff, ORC_F32, g, rows, out);
    }
done:
    free(g); free(u); free(qx);
    return rc;
}

int orc_moe_ffn(int gate_type, const uint8_t* const* gate,
                int up_type, const uint8_t* const* up,
                int down_type, const uint8_t* const* down,
                size_t n_experts, size_t hidden, size_t n_ff,
                const float* x, size_t rows, const int32_t* ids,
                const float* weights, size_t k, int act, float* out) {
    struct moe_ffn_ctx c;
    c.gate_type = gate_type; c.up_type = up_type; c.down_type = down_type;
    c.act = act; c.gate = gate; c.up = up; c.down = down; c.n_ff = n_ff;
    if (act == ORC_Q8_K && (hidden % 256 || n_ff % 256)) return -1;
    return orc_moe_dispatch(x, rows, hidden, n_experts, ids, weights, k, moe_expert_ffn, &c, out);
}

/* ---- the quant crate's own Q4_K ------------------------------------------- */

size_t orc_q4_k_barq_quantize(const float* x, size_t n, uint8_t* out) {
    size_t o = 0;
    for (size_t start = 0; start < n; start += 256) {             /* :27-33 */
        const size_t end = start + 256 < n ? start + 256 : n, len = end - start;
        float mn = INFINITY, mx = -INFINITY;                        /* :39-40, f32::min / f32::max folds */
        for (size_t i = start; i < end; i++) {
            mn = fminf(mn, x[i]);
            mx = fmaxf(mx, x[i]);
        }
        const float scale_min = mn, scale_max = mx - mn;            /* :43-44 */
        const size_t nq = (len + 1) / 2;
        uint8_t* q = out + o + 8;
        memset(q, 0, nq);
        for (size_t i = 0; i < len; i++) {                          /* :49-62 */
            const float normalized = scale_max == 0.0f ? 7.5f : (x[start + i] - scale_min) / scale_max * 15.0f;
            float r = roundf(normalized);                           /* f32::round: half away from zero */
            if (r < 0.0f) r = 0.0f;                                 /* f32::clamp(0, 15) */
            if (r > 15.0f) r = 15.0f;
            const uint8_t qv = r != r ? 0 : (uint8_t)r;            /* `as u8`: NaN -> 0 */
            q[i / 2] |= (uint8_t)(qv << (i % 2 ? 4 : 0));
        }
        memcpy(out + o, &scale_min, 4);                             /* :64-68, little-endian */
        memcpy(out + o + 4, &scale_max, 4);
        o += 8 + nq;
    }
    return o;
}

size_t orc_q4_k_barq_dequantize(const uint8_t* in, size_t in_len, size_t output_size, float* out) {
    const size_t n_blocks = (output_size + 255) / 256;
    size_t off = 0, w = 0;
    for (size_t b = 0; b < n_blocks; b++) {
        if (off + 8 > in_len) break;                                /* :86-88 */
        float scale_min, scale_max;
        memcpy(&scale_min, in + off, 4);
        memcpy(&scale_max, in + off + 4, 4);
        off += 8;
        if (off + 128 > in_len) break;                              /* :108-111 */
        const uint8_t* quants = in + off;
        off += 128;
        for (size_t i = 0; i < 256; i++) {                          /* :117-127 */
            const uint8_t q = (uint8_t)((quants[i / 2] >> (i % 2 ? 4 : 0)) & 0x0F);
            const float t = (float)q / 15.0f;
            const float u = t * scale_max;
            if (w < output_size) out[w] = scale_min + u;
            w++;
        }
    }
    return w < output_size ? w : output_size;                       /* :130 truncate */
}

/* ---- attention ------------------------------------------------------------ */

void orc_rope(const float* x, size_t seq, size_t heads, size_t hd, size_t start_pos, float freq_scale,
              const float* inv_freq, int layout, float* out) {
    /* transformer.rs:525-559: per head, per position, per pair */
    const size_t half = hd / 2;
    for (size_t h = 0; h < heads; h++)
        for (size_t pos = 0; pos < seq; pos++) {
            const size_t src = pos * heads * hd + h * hd, dst = h * seq * hd + pos * hd;
            const size_t abs_pos = start_pos + pos;
            for (size_t i = 0; i < half; i++) {
                const float angle = ((float)abs_pos * freq_scale) * inv_freq[i];
                const float sn = sinf(angle), cs = cosf(angle);
                const size_t i0 = layout == 0 ? 2 * i : i, i1 = layout == 0 ? 2 * i + 1 : i + half;
                const float x0 = x[src + i0], x1 = x[src + i1];
                const float a = x0 * cs, b = x1 * sn, c = x0 * sn, d = x1 * cs;
                out[dst + i0] = a - b;
                out[dst + i1] = c + d;
            }
        }
}

void orc_transpose_heads(const float* x, size_t seq, size_t heads, size_t hd, float* out) {
    for (size_t h = 0; h < heads; h++)
        for (size_t pos = 0; pos < seq; pos++)
            memcpy(out + h * seq * hd + pos * hd, x + pos * heads * hd + h * hd, hd * sizeof(float));
}

void orc_attention(const float* q, const float* kc, const float* vc, size_t head_stride, size_t n_head,
                   size_t n_head_kv, size_t hd, size_t q_len, size_t kv_len, size_t start_pos, float* out) {
    const float scale = sqrtf((float)hd);            /* :311 */
    const float inv_scale = 1.0f / scale;            /* :327 */
    float* scores = (float*)malloc((kv_len ? kv_len : 1) * sizeof(float));
    float* head_out = (float*)malloc(hd * sizeof(float));
    for (size_t h = 0; h < n_head; h++) {
        const size_t kv_h = h * n_head_kv / n_head;   /* :318 */
        const float* q_head = q + h * q_len * hd;
        const float* k_head = kc + kv_h * head_stride;
        const float* v_head = vc + kv_h * head_stride;
        for (size_t i = 0; i < q_len; i++) {
            orc_gemv_f32(k_head, q_head + i * hd, kv_len, hd, scores);   /* :331 */
            for (size_t j = 0; j < kv_len; j++) scores[j] *= inv_scale;
            const size_t valid_len = start_pos + i + 1;                   /* :337-342 */
            for (size_t j = valid_len; j < kv_len; j++) scores[j] = -INFINITY;
            float max_s = -INFINITY;                                      /* :345, f32::max */
            for (size_t j = 0; j < kv_len; j++) max_s = fmaxf(max_s, scores[j]);
            float exp_sum = 0.0f;
            for (size_t j = 0; j < kv_len; j++) {
                scores[j] = expf(scores[j] - max_s);
                exp_sum += scores[j];
            }
            for (size_t j = 0; j < kv_len; j++) scores[j] /= exp_sum;
            orc_gemm_f32(scores, v_head, 1, kv_len, hd, head_out);        /* :355 */
            memcpy(out + i * n_head * hd + h * hd, head_out, hd * sizeof(float));   /* :365-371 */
        }
    }
    free(scores);
    free(head_out);
}
