/*
 * Scalar C restatement of the GGUF / MXFP4 block formats — TEST ORACLE ONLY.
 *
 * Written per element from the block definitions (not from the vectorised
 * restatement in oracle/gguf.py), so that a wrong split, shift or index in either
 * shows up as a mismatch between the two. Only tests/ load this library.
 *
 *   Q8_0 (34 B / 32):  fp16 d @0, int8 q[32] @2;              v = d*q
 *   Q4_K (144 B / 256): fp16 d @0, fp16 dmin @2, s[12] @4, qs[128] @16
 *   Q5_K (176 B / 256): fp16 d @0, fp16 dmin @2, s[12] @4, qh[32] @16, qs[128] @48
 *   Q6_K (210 B / 256): ql[128] @0, qh[64] @128, int8 sc[16] @192, fp16 d @208
 *   MXFP4: byte blocks[n][k/32][(k%32)/2], low nibble for even k; e8m0 scale[n][k/32]
 *
 * Reference semantics: tinyserve/gguf_dequant_torch.py:101-111,118-122,187-249 and
 * tinyserve/mxfp4.py:5-44.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float f16_to_f32(uint16_t h) {
    /* IEEE binary16 -> binary32 from the definition (exact, subnormals kept). */
    int s = (h >> 15) & 1, e = (h >> 10) & 31, m = h & 1023;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(m | 1024), e - 25);
    return s ? -v : v;
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* 6-bit sub-block scale and min j (0..7) of a Q4_K/Q5_K 12-byte field. */
static void k_scale_min(const uint8_t* s, int j, int* sc, int* m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

static float q8_0_elem(const uint8_t* b, int e) {
    return f16_to_f32(rd16(b)) * (float)(int8_t)b[2 + e];
}

static float q4_k_elem(const uint8_t* b, int e) {
    float d = f16_to_f32(rd16(b)), dmin = f16_to_f32(rd16(b + 2));
    int c = e / 64, l = e % 64, q, j, sc, m;
    if (l < 32) { q = b[16 + 32 * c + l] & 15; j = 2 * c; }
    else        { q = b[16 + 32 * c + l - 32] >> 4; j = 2 * c + 1; }
    k_scale_min(b + 4, j, &sc, &m);
    float a = d * (float)sc, bm = dmin * (float)m;
    volatile float prod = a * (float)q; /* exact; keep the reference's two-step form */
    return prod - bm;
}

static float q5_k_elem(const uint8_t* b, int e) {
    float d = f16_to_f32(rd16(b)), dmin = f16_to_f32(rd16(b + 2));
    int c = e / 64, l = e % 64, lo, j, sc, m;
    if (l < 32) { lo = b[48 + 32 * c + l] & 15; }
    else        { lo = b[48 + 32 * c + l - 32] >> 4; }
    j = e / 32;
    int hi = (b[16 + (e % 32)] >> j) & 1;
    int q = lo | (hi << 4);
    k_scale_min(b + 4, j, &sc, &m);
    float a = d * (float)sc, bm = dmin * (float)m;
    volatile float prod = a * (float)q;
    return prod - bm;
}

static float q6_k_elem(const uint8_t* b, int e) {
    int h = e / 128, r = e % 128, t = r / 32, l = r % 32;
    int lo = (b[64 * h + 32 * (t & 1) + l] >> (4 * (t >> 1))) & 15;
    int hi = (b[128 + 32 * h + l] >> (2 * t)) & 3;
    int q = (lo | (hi << 4)) - 32;
    float d = f16_to_f32(rd16(b + 208));
    float ds = d * (float)(int8_t)b[192 + e / 16];
    return ds * (float)q;
}

static int type_info(int type, int* bs, int* ts) {
    switch (type) {
        case 8:  *bs = 32;  *ts = 34;  return 0;
        case 12: *bs = 256; *ts = 144; return 0;
        case 13: *bs = 256; *ts = 176; return 0;
        case 14: *bs = 256; *ts = 210; return 0;
        default: return -1;
    }
}

static float gguf_elem(int type, const uint8_t* data, int64_t i) {
    int bs, ts;
    type_info(type, &bs, &ts);
    const uint8_t* b = data + (i / bs) * ts;
    int e = (int)(i % bs);
    switch (type) {
        case 8:  return q8_0_elem(b, e);
        case 12: return q4_k_elem(b, e);
        case 13: return q5_k_elem(b, e);
        default: return q6_k_elem(b, e);
    }
}

/* Dequantise n_elems (a whole number of blocks) of the flat block stream. */
int oracle_gguf_dequant(int type, const uint8_t* data, int64_t n_elems, float* out) {
    int bs, ts;
    if (type_info(type, &bs, &ts)) return -1;
    if (n_elems % bs) return -2;
    for (int64_t i = 0; i < n_elems; ++i) out[i] = gguf_elem(type, data, i);
    return 0;
}

/* y[n] = sum_k W[n][k] * x[k] with W element (n,k) = flat index n*K+k; double accumulate. */
int oracle_gguf_matvec(int type, const uint8_t* data, const float* x, int64_t N, int64_t K, float* y) {
    int bs, ts;
    if (type_info(type, &bs, &ts)) return -1;
    if ((N * K) % bs) return -2;
    for (int64_t n = 0; n < N; ++n) {
        double acc = 0.0;
        for (int64_t k = 0; k < K; ++k) acc += (double)gguf_elem(type, data, n * K + k) * (double)x[k];
        y[n] = (float)acc;
    }
    return 0;
}

static const float FP4[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                              -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

static float e8m0(uint8_t s) {
    if (s == 255) return INFINITY;
    return ldexpf(1.0f, (int)s - 127);
}

static float mxfp4_elem(const uint8_t* blocks, const uint8_t* scales, int64_t K, int64_t n, int64_t k) {
    int64_t G = K / 32;
    uint8_t byte = blocks[(n * G + k / 32) * 16 + (k % 32) / 2];
    int nib = (k & 1) ? (byte >> 4) : (byte & 15);
    return FP4[nib] * e8m0(scales[n * G + k / 32]);
}

int oracle_mxfp4_dequant(const uint8_t* blocks, const uint8_t* scales, int64_t N, int64_t K, float* out) {
    if (K % 32) return -2;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) out[n * K + k] = mxfp4_elem(blocks, scales, K, n, k);
    return 0;
}

int oracle_mxfp4_matvec(const uint8_t* blocks, const uint8_t* scales, const float* bias, const float* x,
                        int64_t N, int64_t K, float* y) {
    if (K % 32) return -2;
    for (int64_t n = 0; n < N; ++n) {
        double acc = bias ? (double)bias[n] : 0.0;
        for (int64_t k = 0; k < K; ++k) acc += (double)mxfp4_elem(blocks, scales, K, n, k) * (double)x[k];
        y[n] = (float)acc;
    }
    return 0;
}
