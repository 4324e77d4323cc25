/* jam_oracle.c — CPU restatement of jam's quantized-matmul arithmetic. TEST INFRASTRUCTURE ONLY:
 * nothing in the product links or calls it (see jam_oracle.h for what may, and how each part is pinned).
 * Written from the documented math of the reference; reference citations are file:line relative to the
 * qxoticai/qxotic repository root. Compiled with -O2 -fno-fast-math -ffp-contract=off so every f32
 * expression rounds exactly where it is written. */
#include "jam_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ geometry */

int jo_block_elems(int dt) {   /* GGMLType.java:15-26 */
    switch (dt) {
    case JO_F32: case JO_F16: case JO_BF16: return 1;
    case JO_Q4_0: case JO_Q8_0: case JO_MXFP4: return 32;
    case JO_NVFP4: return 64;     /* jam_nvfp4.h:14 */
    case JO_Q1_0: return 128;     /* jam_q1_0.h:8 */
    case JO_Q4_K: case JO_Q5_K: case JO_Q6_K: return 256;
    default: return 0;
    }
}

int jo_block_bytes(int dt) {   /* GGMLType.java:15-26 */
    switch (dt) {
    case JO_F32: return 4;
    case JO_F16: case JO_BF16: return 2;
    case JO_Q4_0: return 18;
    case JO_Q8_0: return 34;
    case JO_MXFP4: return 17;
    case JO_Q4_K: return 144;
    case JO_Q5_K: return 176;
    case JO_Q6_K: return 210;
    case JO_NVFP4: return 36;     /* d[4] UE4M3 + qs[32] */
    case JO_Q1_0: return 18;      /* fp16 d + 16 sign bytes */
    default: return 0;
    }
}

int64_t jo_span_bytes(int dt, int rows, int stride, int row_elems) {   /* GGMLType.java:43-54 */
    int be = jo_block_elems(dt), bb = jo_block_bytes(dt);
    if (!be) return -1;
    return (int64_t)(rows - 1) * (stride / be) * bb + (int64_t)(row_elems / be) * bb;
}

/* ------------------------------------------------------------------ scalar formats */

float jo_half2float(uint16_t h) {   /* jam_fp16.h:8-27: exact IEEE binary16 decode */
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    int e = (h >> 10) & 31;
    uint32_t man = h & 0x3FFu, bits;
    if (e == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else if (e == 0) {
        if (man == 0) {
            bits = sign;
        } else {   /* subnormal: man * 2^-24, normalise */
            int shift = 0;
            while (!(man & 0x400u)) { man <<= 1; shift++; }
            bits = sign | ((uint32_t)(113 - shift) << 23) | ((man & 0x3FFu) << 13);
        }
    } else {
        bits = sign | ((uint32_t)(e + 112) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t jo_float2half(float f) {   /* round-to-nearest-even binary32 -> binary16 */
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);          /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) {                                             /* below 2^-14: subnormal half */
        if (ax < 0x33000000u) return (uint16_t) sign;                   /* < 2^-25 -> 0 */
        int e = (int)(ax >> 23);
        uint32_t man = (ax & 0x7FFFFFu) | 0x800000u;
        int shift = 126 - e;                                            /* 14..24 */
        uint32_t q = man >> shift, rem = man & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((ax - 0x38000000u) >> 13);                            /* rebias exponent */
    uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++;
    return (uint16_t)(sign | q);
}

float jo_e8m0_half(uint8_t e) {   /* jam_mxfp4.h:17-24: 0.5 * 2^(e-127) */
    uint32_t bits = (e == 0) ? 0x00400000u : ((uint32_t) e << 23);
    float s;
    memcpy(&s, &bits, 4);
    return 0.5f * s;
}

static float bf16f(uint16_t h) { uint32_t b = (uint32_t) h << 16; float f; memcpy(&f, &b, 4); return f; }

float jo_ue4m3(uint8_t x) {   /* jam_nvfp4.h:19-25 */
    if (x == 0 || x == 0x7F) return 0.0f;
    int e = (x >> 3) & 0xF, m = x & 0x7;
    return e ? ldexpf(1.0f + (float) m / 8.0f, e - 7) : ldexpf((float) m, -9);
}

uint16_t jo_float2bf16(float f) {   /* round to nearest even on the 16 dropped bits */
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);   /* NaN stays (quiet) NaN */
    x += 0x7FFFu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

static const int8_t kMxfp4Codes[16] = { 0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12 };

/* Q4_K / Q5_K packed 6-bit scales and mins (jam/jam-native/src/jam_kquant.h:26-33). */
static void q4k_scales(const uint8_t* b, int sc[8], int mn[8]) {
    for (int j = 0; j < 4; j++) {
        sc[j] = b[j] & 63;
        mn[j] = b[j + 4] & 63;
        sc[j + 4] = (b[j + 8] & 15) | ((b[j] >> 6) << 4);
        mn[j + 4] = (b[j + 8] >> 4) | ((b[j + 4] >> 6) << 4);
    }
}

/* Q6_K element -> (6-bit code, int8 scale index) (jam_kernels_generic.c:217-252). */
static int q6k_code(const uint8_t* blk, int e, int* sidx) {
    int h = e / 128, j = (e % 128) / 32, l = e % 32;
    uint8_t qlb = blk[64 * h + (j & 1) * 32 + l];
    int nib = j < 2 ? (qlb & 15) : (qlb >> 4);
    int hi = (blk[128 + 32 * h + l] >> (2 * j)) & 3;
    *sidx = 8 * h + 2 * j + l / 16;
    return nib | (hi << 4);
}

/* ------------------------------------------------------------------ dequantization */

void jo_dequant_row_f64(int dt, const uint8_t* w, int k, double* out) {
    int be = jo_block_elems(dt), bb = jo_block_bytes(dt);
    for (int B = 0; B < k / be; B++, w += bb, out += be) {
        switch (dt) {
        case JO_F32: { float f; memcpy(&f, w, 4); out[0] = f; break; }
        case JO_F16: out[0] = jo_half2float((uint16_t)(w[0] | (w[1] << 8))); break;
        case JO_BF16: out[0] = bf16f((uint16_t)(w[0] | (w[1] << 8))); break;
        case JO_Q8_0: {   /* generic.c:42-67 */
            double d = jo_half2float((uint16_t)(w[0] | (w[1] << 8)));
            for (int e = 0; e < 32; e++) out[e] = d * (int8_t) w[2 + e];
            break;
        }
        case JO_Q4_0: {   /* generic.c:291-321 */
            double d = jo_half2float((uint16_t)(w[0] | (w[1] << 8)));
            for (int e = 0; e < 16; e++) {
                out[e] = d * ((w[2 + e] & 15) - 8);
                out[e + 16] = d * ((w[2 + e] >> 4) - 8);
            }
            break;
        }
        case JO_MXFP4: {   /* generic.c:96-126 */
            double s = jo_e8m0_half(w[0]);
            for (int e = 0; e < 16; e++) {
                out[e] = s * kMxfp4Codes[w[1 + e] & 15];
                out[e + 16] = s * kMxfp4Codes[w[1 + e] >> 4];
            }
            break;
        }
        case JO_Q4_K: {   /* generic.c:183-215 */
            double d = jo_half2float((uint16_t)(w[0] | (w[1] << 8)));
            double dmin = jo_half2float((uint16_t)(w[2] | (w[3] << 8)));
            int sc[8], mn[8];
            q4k_scales(w + 4, sc, mn);
            for (int g = 0; g < 4; g++)
                for (int e = 0; e < 32; e++) {
                    uint8_t q = w[16 + 32 * g + e];
                    out[64 * g + e] = d * sc[2 * g] * (q & 15) - dmin * mn[2 * g];
                    out[64 * g + 32 + e] = d * sc[2 * g + 1] * (q >> 4) - dmin * mn[2 * g + 1];
                }
            break;
        }
        case JO_Q5_K: {   /* generic.c:254-289 */
            double d = jo_half2float((uint16_t)(w[0] | (w[1] << 8)));
            double dmin = jo_half2float((uint16_t)(w[2] | (w[3] << 8)));
            int sc[8], mn[8];
            q4k_scales(w + 4, sc, mn);
            const uint8_t* qh = w + 16;
            const uint8_t* qs = w + 48;
            for (int g = 0; g < 4; g++)
                for (int e = 0; e < 32; e++) {
                    int lo = (qs[32 * g + e] & 15) | (((qh[e] >> (2 * g)) & 1) << 4);
                    int hi = (qs[32 * g + e] >> 4) | (((qh[e] >> (2 * g + 1)) & 1) << 4);
                    out[64 * g + e] = d * sc[2 * g] * lo - dmin * mn[2 * g];
                    out[64 * g + 32 + e] = d * sc[2 * g + 1] * hi - dmin * mn[2 * g + 1];
                }
            break;
        }
        case JO_Q6_K: {   /* generic.c:217-252 */
            double d = jo_half2float((uint16_t)(w[208] | (w[209] << 8)));
            for (int e = 0; e < 256; e++) {
                int s;
                int q = q6k_code(w, e, &s);
                out[e] = d * (int8_t) w[192 + s] * (q - 32);
            }
            break;
        }
        case JO_NVFP4: {   /* generic.c:128-165: sub-block s byte s*8+j: low nibble elem 16s+j, high 16s+8+j */
            for (int sb = 0; sb < 4; sb++) {
                double d = jo_ue4m3(w[sb]);
                for (int j = 0; j < 8; j++) {
                    uint8_t b = w[4 + 8 * sb + j];
                    out[16 * sb + j] = d * kMxfp4Codes[b & 15];
                    out[16 * sb + 8 + j] = d * kMxfp4Codes[b >> 4];
                }
            }
            break;
        }
        case JO_Q1_0: {   /* jam_q1_0.h:16-27: bit j (LSB-first, byte j/8) ? +d : -d */
            double d = jo_half2float((uint16_t)(w[0] | (w[1] << 8)));
            for (int e = 0; e < 128; e++) out[e] = ((w[2 + (e >> 3)] >> (e & 7)) & 1) ? d : -d;
            break;
        }
        default: break;
        }
    }
}

void jo_dequant_row(int dt, const uint8_t* w, int k, float* out) {
    double* tmp = (double*) malloc(sizeof(double) * (size_t) k);
    jo_dequant_row_f64(dt, w, k, tmp);
    for (int i = 0; i < k; i++) out[i] = (float) tmp[i];
    free(tmp);
}

/* ------------------------------------------------------------------ the repo's own weight quantizers */

static float amax_of(const float* x, int n) {
    float m = 0.0f;
    for (int i = 0; i < n; i++) { float a = fabsf(x[i]); if (a > m) m = a; }
    return m;
}

static void put_half(uint8_t* p, float f) { uint16_t h = jo_float2half(f); p[0] = (uint8_t) h; p[1] = (uint8_t)(h >> 8); }

static int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

void jo_quantize_row(int dt, const float* x, int k, uint8_t* out) {
    int be = jo_block_elems(dt), bb = jo_block_bytes(dt);
    for (int B = 0; B < k / be; B++, x += be, out += bb) {
        memset(out, 0, (size_t) bb);
        switch (dt) {
        case JO_Q8_0: {   /* d = amax/127 (fp16 RNE), q = rint(x/d) */
            float d = amax_of(x, 32) / 127.0f;
            put_half(out, d);
            float id = d > 0.0f ? 1.0f / d : 0.0f;
            for (int e = 0; e < 32; e++) out[2 + e] = (uint8_t)(int8_t) clampi((int) lrintf(x[e] * id), -128, 127);
            break;
        }
        case JO_Q4_0: {   /* ggml convention: signed max mx, d = mx/-8, q = min(15, floor(x/d + 8.5)) */
            float mx = 0.0f, am = 0.0f;
            for (int e = 0; e < 32; e++) if (fabsf(x[e]) > am) { am = fabsf(x[e]); mx = x[e]; }
            float d = mx / -8.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
            put_half(out, d);
            for (int e = 0; e < 16; e++) {
                int q0 = clampi((int) floorf(x[e] * id + 8.5f), 0, 15);
                int q1 = clampi((int) floorf(x[e + 16] * id + 8.5f), 0, 15);
                out[2 + e] = (uint8_t)(q0 | (q1 << 4));
            }
            break;
        }
        case JO_MXFP4: {   /* shared exponent floor(log2 amax) - 2, nearest E2M1 magnitude */
            static const float mag[8] = { 0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f };
            float am = amax_of(x, 32);
            int e8 = 127;
            if (am > 0.0f) e8 = clampi((int) floorf(log2f(am)) - 2 + 127, 1, 254);
            out[0] = (uint8_t) e8;
            float scale = ldexpf(1.0f, e8 - 127);
            for (int e = 0; e < 32; e++) {
                float v = x[e] / scale, a = fabsf(v);
                int best = 0;
                for (int i = 1; i < 8; i++) if (fabsf(a - mag[i]) < fabsf(a - mag[best])) best = i;
                int code = best | ((v < 0.0f && best) ? 8 : 0);
                if (e < 16) out[1 + e] |= (uint8_t) code;
                else out[1 + e - 16] |= (uint8_t)(code << 4);
            }
            break;
        }
        case JO_Q4_K: {   /* 8 sub-blocks: (scale, min) per 32, 6-bit sub-scales under fp16 d/dmin */
            float sub_s[8], sub_m[8], ms = 0.0f, mm = 0.0f;
            for (int s = 0; s < 8; s++) {
                float lo = x[32 * s], hi = x[32 * s];
                for (int e = 1; e < 32; e++) { float v = x[32 * s + e]; lo = v < lo ? v : lo; hi = v > hi ? v : hi; }
                if (lo > 0.0f) lo = 0.0f;
                sub_s[s] = (hi - lo) / 15.0f;
                sub_m[s] = -lo;
                ms = sub_s[s] > ms ? sub_s[s] : ms;
                mm = sub_m[s] > mm ? sub_m[s] : mm;
            }
            float d = jo_half2float(jo_float2half(ms / 63.0f)), dmin = jo_half2float(jo_float2half(mm / 63.0f));
            put_half(out, ms / 63.0f);
            put_half(out + 2, mm / 63.0f);
            int sc[8], mn[8];
            for (int s = 0; s < 8; s++) {
                sc[s] = d > 0.0f ? clampi((int) lrintf(sub_s[s] / d), 0, 63) : 0;
                mn[s] = dmin > 0.0f ? clampi((int) lrintf(sub_m[s] / dmin), 0, 63) : 0;
            }
            uint8_t* b = out + 4;
            for (int j = 0; j < 4; j++) {
                b[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
                b[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
                b[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
            }
            for (int s = 0; s < 8; s++) {
                float ds = d * sc[s], ms_ = dmin * mn[s];
                for (int e = 0; e < 32; e++) {
                    int q = ds > 0.0f ? clampi((int) lrintf((x[32 * s + e] + ms_) / ds), 0, 15) : 0;
                    int g = s / 2, byte = 16 + 32 * g + e;
                    out[byte] |= (uint8_t)((s & 1) ? (q << 4) : q);
                }
            }
            break;
        }
        case JO_F32: memcpy(out, x, 4); break;
        case JO_F16: put_half(out, x[0]); break;
        case JO_BF16: { uint16_t h = jo_float2bf16(x[0]); out[0] = (uint8_t) h; out[1] = (uint8_t)(h >> 8); break; }
        case JO_Q5_K: {   /* as Q4_K with 32 levels: the 5th bit of sub-block 2g/2g+1 in bit 2g/2g+1 of qh[e] */
            float sub_s[8], sub_m[8], ms = 0.0f, mm = 0.0f;
            for (int s = 0; s < 8; s++) {
                float lo = x[32 * s], hi = x[32 * s];
                for (int e = 1; e < 32; e++) { float v = x[32 * s + e]; lo = v < lo ? v : lo; hi = v > hi ? v : hi; }
                if (lo > 0.0f) lo = 0.0f;
                sub_s[s] = (hi - lo) / 31.0f;
                sub_m[s] = -lo;
                ms = sub_s[s] > ms ? sub_s[s] : ms;
                mm = sub_m[s] > mm ? sub_m[s] : mm;
            }
            float d = jo_half2float(jo_float2half(ms / 63.0f)), dmin = jo_half2float(jo_float2half(mm / 63.0f));
            put_half(out, ms / 63.0f);
            put_half(out + 2, mm / 63.0f);
            int sc[8], mn[8];
            for (int s = 0; s < 8; s++) {
                sc[s] = d > 0.0f ? clampi((int) lrintf(sub_s[s] / d), 0, 63) : 0;
                mn[s] = dmin > 0.0f ? clampi((int) lrintf(sub_m[s] / dmin), 0, 63) : 0;
            }
            uint8_t* b = out + 4;
            for (int j = 0; j < 4; j++) {
                b[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
                b[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
                b[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
            }
            for (int s = 0; s < 8; s++) {
                float ds = d * sc[s], ms_ = dmin * mn[s];
                for (int e = 0; e < 32; e++) {
                    int q = ds > 0.0f ? clampi((int) lrintf((x[32 * s + e] + ms_) / ds), 0, 31) : 0;
                    int g = s / 2;
                    out[48 + 32 * g + e] |= (uint8_t)((s & 1) ? ((q & 15) << 4) : (q & 15));
                    out[16 + e] |= (uint8_t)((q >> 4) << s);
                }
            }
            break;
        }
        case JO_NVFP4: {   /* per 16: the UE4M3 scale nearest amax/12, then the nearest code of kv = 2·e2m1 */
            for (int sb = 0; sb < 4; sb++) {
                const float* v = x + 16 * sb;
                float target = amax_of(v, 16) / 12.0f, best = 1e30f;
                int code = 0;
                for (int c = 1; c < 127; c++) {
                    float dv = fabsf(jo_ue4m3((uint8_t) c) - target);
                    if (c != 0x7F && dv < best) { best = dv; code = c; }
                }
                if (target == 0.0f) code = 0;
                out[sb] = (uint8_t) code;
                float sc = jo_ue4m3((uint8_t) code);
                for (int j = 0; j < 16; j++) {
                    int nib = 0;
                    if (sc > 0.0f) {
                        float t = v[j] / sc, bd = 1e30f;
                        for (int c = 0; c < 16; c++) {
                            float dv = fabsf((float) kMxfp4Codes[c] - t);
                            if (dv < bd) { bd = dv; nib = c; }
                        }
                    }
                    uint8_t* byte = out + 4 + 8 * sb + (j & 7);
                    *byte |= (uint8_t)(j < 8 ? nib : nib << 4);
                }
            }
            break;
        }
        case JO_Q1_0: {   /* d = mean |x| (fp16), bit = x >= 0 */
            float s = 0.0f;
            for (int e = 0; e < 128; e++) s += fabsf(x[e]);
            put_half(out, s / 128.0f);
            for (int e = 0; e < 128; e++)
                if (x[e] >= 0.0f) out[2 + (e >> 3)] |= (uint8_t)(1u << (e & 7));
            break;
        }
        case JO_Q6_K: {   /* 16 sub-blocks of 16: int8 sub-scale under fp16 d, codes q+32 in 0..63 */
            float sub[16], ms = 0.0f;
            for (int s = 0; s < 16; s++) { sub[s] = amax_of(x + 16 * s, 16) / 31.0f; ms = sub[s] > ms ? sub[s] : ms; }
            float d = jo_half2float(jo_float2half(ms / 127.0f));
            put_half(out + 208, ms / 127.0f);
            int sc[16];
            for (int s = 0; s < 16; s++) {
                sc[s] = d > 0.0f ? clampi((int) lrintf(sub[s] / d), -128, 127) : 0;
                out[192 + s] = (uint8_t)(int8_t) sc[s];
            }
            for (int e = 0; e < 256; e++) {
                int h = e / 128, j = (e % 128) / 32, l = e % 32, s = 8 * h + 2 * j + l / 16;
                float ds = d * sc[s];
                int q = ds != 0.0f ? clampi((int) lrintf(x[e] / ds), -32, 31) : 0;
                int u = q + 32;
                uint8_t* qlb = out + 64 * h + (j & 1) * 32 + l;
                *qlb |= (uint8_t)(j < 2 ? (u & 15) : ((u & 15) << 4));
                out[128 + 32 * h + l] |= (uint8_t)((u >> 4) << (2 * j));
            }
            break;
        }
        default: break;
        }
    }
}

/* ------------------------------------------------------------------ activation quantizers */

void jo_quant_f1(const float* x, int k, int8_t* q, float* d, float* asum) {   /* generic.c:71-94 */
    for (int b = 0; b < k / 32; b++) {
        const float* v = x + 32 * b;
        float amax = 0.0f;
        for (int e = 0; e < 32; e++) { float a = fabsf(v[e]); if (a > amax) amax = a; }
        float db = amax / 127.0f;
        float id = db > 0.0f ? 1.0f / db : 0.0f;
        int sum = 0;
        for (int e = 0; e < 32; e++) {
            long r = lrintf(v[e] * id);
            int t = r > 127 ? 127 : r < -128 ? -128 : (int) r;
            q[32 * b + e] = (int8_t) t;
            sum += t;
        }
        d[b] = db;
        if (asum) asum[b] = (float) sum;
    }
}

static float tree16(const float* v) {   /* _mm512_reduce_add_ps: fold 8, 4, 2, 1 */
    float t8[8], t4[4], t2[2];
    for (int i = 0; i < 8; i++) t8[i] = v[i + 8] + v[i];
    for (int i = 0; i < 4; i++) t4[i] = t8[i + 4] + t8[i];
    for (int i = 0; i < 2; i++) t2[i] = t4[i] + t4[i + 2];
    return t2[0] + t2[1];
}

static int sat8_rne(float f) {   /* _mm512_cvtps_epi32 (RNE; NaN/overflow -> INT_MIN) then cvtsepi32_epi8 */
    if (!(f > -2147483648.0f && f < 2147483648.0f)) return -128;
    float r = rintf(f);
    if (r > 127.0f) return 127;
    if (r < -128.0f) return -128;
    return (int) r;
}

void jo_quant_f2(const float* x, int k, int8_t* q, float* d, float* xs) {   /* q4k_avx512.c:25-37 */
    for (int b = 0; b < k / 32; b++) {
        const float* v = x + 32 * b;
        float mx = 0.0f;
        for (int e = 0; e < 32; e++) { float a = fabsf(v[e]); if (a > mx) mx = a; }
        d[b] = mx / 127.0f;
        float inv = mx > 0.0f ? 127.0f / mx : 0.0f;
        xs[2 * b] = tree16(v);
        xs[2 * b + 1] = tree16(v + 16);
        for (int e = 0; e < 32; e++) q[32 * b + e] = (int8_t) sat8_rne(v[e] * inv);
    }
}

/* ------------------------------------------------------------------ int8 pipeline */

static float h2f_at(const uint8_t* p) { return jo_half2float((uint16_t)(p[0] | (p[1] << 8))); }

/* One weight row against one quantized activation row, flavour 1 (n<8 kernels).
 *   Q8_0  : Σ_b fl(d·ad)·Σq·aq                     (jam_gemm_q256.inc:28-36; avx512.c:374-390)
 *   Q4_0  : Σ_b fl(d·ad)·Σ(nib-8)·aq                (jam_decode_x86_256.h:22-30 + q256 engine)
 *   MXFP4 : Σ_b fl(dhalf·ad)·Σcode·aq               (jam_decode_x86_256.h:33-42 + q256 engine)
 *   Q4_K  : Σ_s fl(fl(ad·sc)·d)·Σnib·aq − dmin·mn·fl(asum·ad)   (q4k_avx512.c:956-1054)
 *   Q6_K  : Σ_blk ad·(fl(d·sc0)·dot0 + fl(d·sc1)·dot1), dots over (q6-32)·aq  (kquant_sse3.c:125-169) */
static double row_f1(int dt, const uint8_t* w, const int8_t* aq, const float* ad, const float* as, int k) {
    double acc = 0.0;
    if (dt == JO_Q8_0 || dt == JO_Q4_0 || dt == JO_MXFP4) {
        int bb = jo_block_bytes(dt);
        for (int b = 0; b < k / 32; b++, w += bb) {
            const int8_t* a = aq + 32 * b;
            int dot = 0;
            float sw;
            if (dt == JO_Q8_0) {
                sw = h2f_at(w);
                for (int e = 0; e < 32; e++) dot += (int8_t) w[2 + e] * a[e];
            } else if (dt == JO_Q4_0) {
                sw = h2f_at(w);
                for (int e = 0; e < 16; e++) dot += ((w[2 + e] & 15) - 8) * a[e] + ((w[2 + e] >> 4) - 8) * a[e + 16];
            } else {
                sw = jo_e8m0_half(w[0]);
                for (int e = 0; e < 16; e++) dot += kMxfp4Codes[w[1 + e] & 15] * a[e] + kMxfp4Codes[w[1 + e] >> 4] * a[e + 16];
            }
            float s = sw * ad[b];
            acc += (double) s * dot;
        }
        return acc;
    }
    if (dt == JO_Q4_K) {
        for (int B = 0; B < k / 256; B++, w += 144) {
            float d = h2f_at(w), dmin = h2f_at(w + 2);
            int sc[8], mn[8];
            q4k_scales(w + 4, sc, mn);
            for (int s = 0; s < 8; s++) {
                int g = s / 2, bi = 8 * B + s;
                const int8_t* a = aq + 32 * bi;
                int dot = 0;
                for (int e = 0; e < 32; e++) {
                    uint8_t q = w[16 + 32 * g + e];
                    dot += ((s & 1) ? (q >> 4) : (q & 15)) * a[e];
                }
                float f = (ad[bi] * (float) sc[s]) * d;
                float asd = as[bi] * ad[bi];
                acc += (double) f * dot - (double) dmin * ((double) mn[s] * asd);
            }
        }
        return acc;
    }
    if (dt == JO_Q6_K) {
        for (int B = 0; B < k / 256; B++, w += 210) {
            float d = h2f_at(w + 208);
            for (int t = 0; t < 8; t++) {   /* 32-blocks of the super-block */
                int bi = 8 * B + t, dot[2] = { 0, 0 }, si[2] = { 0, 0 };
                for (int e = 0; e < 32; e++) {
                    int s;
                    int q = q6k_code(w, 32 * t + e, &s);
                    dot[e / 16] += (q - 32) * aq[32 * bi + e];
                    si[e / 16] = s;
                }
                float s0 = d * (float)(int8_t) w[192 + si[0]], s1 = d * (float)(int8_t) w[192 + si[1]];
                acc += (double) ad[bi] * ((double) s0 * dot[0] + (double) s1 * dot[1]);
            }
        }
        return acc;
    }
    if (dt == JO_Q5_K) {   /* jam_mm_q5k_sse3 (kquant_sse3.c:70-121): ad·(fl(dl·dot) − fl(ml·asum)) per 32 */
        for (int B = 0; B < k / 256; B++, w += 176) {
            float d = h2f_at(w), dmin = h2f_at(w + 2);
            int sc[8], mn[8];
            q4k_scales(w + 4, sc, mn);
            const uint8_t* qh = w + 16;
            const uint8_t* qs = w + 48;
            for (int s = 0; s < 8; s++) {
                int g = s / 2, bi = 8 * B + s, dot = 0;
                for (int e = 0; e < 32; e++) {
                    uint8_t q = qs[32 * g + e];
                    int q5 = ((s & 1) ? (q >> 4) : (q & 15)) | (((qh[e] >> s) & 1) << 4);
                    dot += q5 * aq[32 * bi + e];
                }
                float dl = d * (float) sc[s], ml = dmin * (float) mn[s];
                float t = dl * (float) dot - ml * as[bi];
                acc += (double)(ad[bi] * t);
            }
        }
        return acc;
    }
    if (dt == JO_NVFP4) {   /* jam_mm_nvfp4_avx512 (avx512bw.c:111-142): Σ_s dot_s·fl(ue4m3(d_s)·ad) per 16 */
        for (int bb = 0; bb < k / 64; bb++, w += 36) {
            for (int sb = 0; sb < 4; sb++) {
                int dot = 0;
                for (int j = 0; j < 8; j++) {
                    uint8_t b = w[4 + 8 * sb + j];
                    dot += kMxfp4Codes[b & 15] * aq[64 * bb + 16 * sb + j] + kMxfp4Codes[b >> 4] * aq[64 * bb + 16 * sb + 8 + j];
                }
                float sc = jo_ue4m3(w[sb]) * ad[2 * bb + sb / 2];
                acc += (double) sc * dot;
            }
        }
        return acc;
    }
    if (dt == JO_Q1_0) {   /* jam_mm_q1_0_avx2 (q1_0_avx2.c:45-86): d·Σ_K fma(ad_K, Σ±q, ·) per 128 */
        for (int bb = 0; bb < k / 128; bb++, w += 18) {
            float fb = 0.0f;
            for (int K = 0; K < 4; K++) {
                int bi = 4 * bb + K, dot = 0;
                for (int e = 0; e < 32; e++) {
                    int el = 32 * K + e;
                    int bit = (w[2 + (el >> 3)] >> (el & 7)) & 1;
                    dot += bit ? aq[32 * bi + e] : -aq[32 * bi + e];
                }
                fb = fmaf(ad[bi], (float) dot, fb);
            }
            acc += (double) h2f_at(w) * fb;
        }
        return acc;
    }
    return 0.0;
}

/* Flavour 2 (n>=8 bands, F2 activations with exact per-16 float sums).
 *   Q8_0  : Σ_b fl(d·dx)·Σq·xq                                   (q4k_avx512.c:321-362)
 *   Q4_0  : Σ_b fl(d·dx)·Σnib·xq − fl(8d)·fl(xs0+xs1)           (q4k_avx512.c:424-480)
 *   MXFP4 : Σ_b fl(dhalf·dx)·Σcode·xq                           (q4k_avx512.c:662-711)
 *   Q4_K  : Σ_s fl(fl(d·sc)·dx)·Σnib·xq − fl(dmin·mn)·fl(xs0+xs1) (q4k_avx512.c:50-95)
 *   Q6_K  : Σ_t fl(fl(d·sc_t)·dx)·Σq6·xq − fl(d·sc_t)·fl(32·xs_t)   (q4k_avx512.c:192-236) */
static double row_f2(int dt, const uint8_t* w, const int8_t* xq, const float* dx, const float* xs, int k) {
    double acc = 0.0;
    if (dt == JO_Q8_0 || dt == JO_Q4_0 || dt == JO_MXFP4) {
        int bb = jo_block_bytes(dt);
        for (int b = 0; b < k / 32; b++, w += bb) {
            const int8_t* a = xq + 32 * b;
            int dot = 0;
            if (dt == JO_Q8_0) {
                for (int e = 0; e < 32; e++) dot += (int8_t) w[2 + e] * a[e];
                acc += (double)(h2f_at(w) * dx[b]) * dot;
            } else if (dt == JO_Q4_0) {
                for (int e = 0; e < 16; e++) dot += (w[2 + e] & 15) * a[e] + (w[2 + e] >> 4) * a[e + 16];
                float d = h2f_at(w);
                acc += (double)(d * dx[b]) * dot - (double)(8.0f * d) * (double)(xs[2 * b] + xs[2 * b + 1]);
            } else {
                for (int e = 0; e < 16; e++) dot += kMxfp4Codes[w[1 + e] & 15] * a[e] + kMxfp4Codes[w[1 + e] >> 4] * a[e + 16];
                acc += (double)(jo_e8m0_half(w[0]) * dx[b]) * dot;
            }
        }
        return acc;
    }
    if (dt == JO_Q4_K) {
        for (int B = 0; B < k / 256; B++, w += 144) {
            float d = h2f_at(w), dmin = h2f_at(w + 2);
            int sc[8], mn[8];
            q4k_scales(w + 4, sc, mn);
            for (int s = 0; s < 8; s++) {
                int g = s / 2, bi = 8 * B + s;
                int dot = 0;
                for (int e = 0; e < 32; e++) {
                    uint8_t q = w[16 + 32 * g + e];
                    dot += ((s & 1) ? (q >> 4) : (q & 15)) * xq[32 * bi + e];
                }
                float dw = d * (float) sc[s], mw = dmin * (float) mn[s];
                acc += (double)(dw * dx[bi]) * dot - (double) mw * (double)(xs[2 * bi] + xs[2 * bi + 1]);
            }
        }
        return acc;
    }
    if (dt == JO_Q6_K) {
        for (int B = 0; B < k / 256; B++, w += 210) {
            float d = h2f_at(w + 208);
            for (int t = 0; t < 16; t++) {   /* 16-element groups */
                int dot = 0, s = 0;
                for (int e = 0; e < 16; e++) {
                    int q = q6k_code(w, 16 * t + e, &s);
                    dot += q * xq[256 * B + 16 * t + e];
                }
                float dw = d * (float)(int8_t) w[192 + s];
                int bi = 8 * B + t / 2;
                acc += (double)(dw * dx[bi]) * dot - (double) dw * (double)(32.0f * xs[16 * B + t]);
            }
        }
        return acc;
    }
    if (dt == JO_Q5_K) {   /* q5k_block16 (q4k_avx512.c:798-811): fl(fl(d·sc)·dx)·Σq5·xq − fl(dmin·mn)·fl(xs0+xs1) */
        for (int B = 0; B < k / 256; B++, w += 176) {
            float d = h2f_at(w), dmin = h2f_at(w + 2);
            int sc[8], mn[8];
            q4k_scales(w + 4, sc, mn);
            const uint8_t* qh = w + 16;
            const uint8_t* qs = w + 48;
            for (int s = 0; s < 8; s++) {
                int g = s / 2, bi = 8 * B + s, dot = 0;
                for (int e = 0; e < 32; e++) {
                    uint8_t q = qs[32 * g + e];
                    int q5 = ((s & 1) ? (q >> 4) : (q & 15)) | (((qh[e] >> s) & 1) << 4);
                    dot += q5 * xq[32 * bi + e];
                }
                float dw = d * (float) sc[s], mw = dmin * (float) mn[s];
                acc += (double)(dw * dx[bi]) * dot - (double) mw * (double)(xs[2 * bi] + xs[2 * bi + 1]);
            }
        }
        return acc;
    }
    if (dt == JO_Q1_0) {   /* q1_0_block16 (q4k_avx512.c:580-598): fl(d·fl(2·dx))·Σbit·xq − d·fl(xs0+xs1) */
        for (int bb = 0; bb < k / 128; bb++, w += 18) {
            float d = h2f_at(w);
            for (int K = 0; K < 4; K++) {
                int bi = 4 * bb + K, dot = 0;
                for (int e = 0; e < 32; e++) {
                    int el = 32 * K + e;
                    if ((w[2 + (el >> 3)] >> (el & 7)) & 1) dot += xq[32 * bi + e];
                }
                acc += (double)(d * (2.0f * dx[bi])) * dot - (double) d * (double)(xs[2 * bi] + xs[2 * bi + 1]);
            }
        }
        return acc;
    }
    return 0.0;
}

static int int8_supported(int dt) {
    return dt == JO_Q8_0 || dt == JO_Q4_0 || dt == JO_MXFP4 || dt == JO_Q4_K || dt == JO_Q6_K || dt == JO_Q5_K ||
           dt == JO_NVFP4 || dt == JO_Q1_0;
}

/* jam's block-alignment rule per dtype (jam.c:665-685, 752): k on the block for every quantized dtype;
 * ldw on it too for the 32-element types and Q1_0, while the K-quants and NVFP4 take the row stride as
 * (ldw / block) blocks. */
static int aligned(int dt, int ldw, int k) {
    int be = jo_block_elems(dt);
    if (k % be) return 0;
    if (dt == JO_Q4_K || dt == JO_Q5_K || dt == JO_Q6_K || dt == JO_NVFP4) return 1;
    return ldw % be == 0;
}

/* Exact float dot of one dequantized weight row with an f32 activation row (double accumulation): the
 * "<16-row tail: scalar exact dot" every n>=8 band runs on its last m%16 rows (q4k_avx512.c:185-188,
 * 314-317, 417-420, 551-554, 654-657, 790-793), whose own f32 order differs only by rounding. */
static double row_float(int dt, const uint8_t* w, const float* x, int k) {
    double* row = (double*) malloc(sizeof(double) * (size_t) k);
    jo_dequant_row_f64(dt, w, k, row);
    double s = 0.0;
    for (int e = 0; e < k; e++) s += row[e] * x[e];
    free(row);
    return s;
}

int jo_mm_int8(int dt, const uint8_t* w, int ldw, const float* a, int lda, float* c, int ldc,
               int m, int n, int k, int flavour) {
    if (!int8_supported(dt) || !aligned(dt, ldw, k)) return -1;
    /* flavour 0 = jam's own routing on an AVX-512-VNNI host (jam.c:469-499, 544-560, 682-730): n < 8 runs
     * F1 on every row; n >= 8 runs the 16-row F2 bands and leaves the last m % 16 rows to a float dot.
     * NVFP4 has no band: run_quant's F1 kernel takes every n (jam.c:662-668). */
    const int jam_rule = flavour == 0;
    if (dt == JO_NVFP4 && flavour == 2) return -1;
    if (flavour == 0) flavour = n < 8 || dt == JO_NVFP4 ? 1 : 2;
    const int m_int8 = jam_rule && flavour == 2 ? m - m % 16 : m;
    int nb = k / 32;
    int8_t* q = (int8_t*) malloc((size_t) n * k);
    float* d = (float*) malloc(sizeof(float) * (size_t) n * nb);
    float* s = (float*) malloc(sizeof(float) * (size_t) n * nb * 2);
    for (int j = 0; j < n; j++) {
        if (flavour == 1) jo_quant_f1(a + (size_t) j * lda, k, q + (size_t) j * k, d + (size_t) j * nb, s + (size_t) j * nb);
        else jo_quant_f2(a + (size_t) j * lda, k, q + (size_t) j * k, d + (size_t) j * nb, s + (size_t) j * nb * 2);
    }
    int64_t wstride = (int64_t)(ldw / jo_block_elems(dt)) * jo_block_bytes(dt);
    for (int i = 0; i < m; i++) {
        const uint8_t* wr = w + (int64_t) i * wstride;
        for (int j = 0; j < n; j++) {
            double v = i >= m_int8 ? row_float(dt, wr, a + (size_t) j * lda, k)
                : flavour == 1
                ? row_f1(dt, wr, q + (size_t) j * k, d + (size_t) j * nb, s + (size_t) j * nb, k)
                : row_f2(dt, wr, q + (size_t) j * k, d + (size_t) j * nb, s + (size_t) j * nb * 2, k);
            c[(size_t) j * ldc + i] = (float) v;
        }
    }
    free(q);
    free(d);
    free(s);
    return 0;
}

int jo_bf16_rounds_activations(int n, int k) {   /* jam.c:622-652 on an AVX-512-BF16 host */
    return (n >= 8 && k % 2 == 0) || k % 32 == 0;
}

int jo_mm_dense(int dt, const uint8_t* w, int ldw, const float* a, int lda, float* c, int ldc, int m, int n, int k) {
    if (dt != JO_F32 && dt != JO_F16 && dt != JO_BF16) return -1;
    const int es = jo_block_bytes(dt), rnd = dt == JO_BF16 && jo_bf16_rounds_activations(n, k);
    double* row = (double*) malloc(sizeof(double) * (size_t) k);
    double* x = (double*) malloc(sizeof(double) * (size_t) k);
    for (int j = 0; j < n; j++) {
        const float* aj = a + (size_t) j * lda;
        for (int e = 0; e < k; e++) x[e] = rnd ? bf16f(jo_float2bf16(aj[e])) : aj[e];
        for (int i = 0; i < m; i++) {
            jo_dequant_row_f64(dt, w + (int64_t) i * ldw * es, k, row);
            double s = 0.0;
            for (int e = 0; e < k; e++) s += row[e] * x[e];
            c[(size_t) j * ldc + i] = (float) s;
        }
    }
    free(row);
    free(x);
    return 0;
}

int jo_mm_ref(int dt, const uint8_t* w, int ldw, const float* a, int lda, double* c, double* sumabs,
              int ldc, int m, int n, int k) {
    int be = jo_block_elems(dt);
    if (!be || k % be || (be > 1 && !aligned(dt, ldw, k))) return -1;
    int64_t wstride = (int64_t)(ldw / be) * jo_block_bytes(dt);
    double* row = (double*) malloc(sizeof(double) * (size_t) k);
    for (int i = 0; i < m; i++) {
        jo_dequant_row_f64(dt, w + (int64_t) i * wstride, k, row);
        for (int j = 0; j < n; j++) {
            const float* x = a + (size_t) j * lda;
            double s = 0.0, sa = 0.0;
            for (int e = 0; e < k; e++) { double p = row[e] * x[e]; s += p; sa += fabs(p); }
            if (c) c[(size_t) j * ldc + i] = s;
            if (sumabs) sumabs[(size_t) j * ldc + i] = sa;
        }
    }
    free(row);
    return 0;
}

/* ------------------------------------------------------------------ generators */

static uint64_t splitmix64(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static double unit_open(uint64_t* s) { return ((double)(splitmix64(s) >> 11) + 0.5) * (1.0 / 9007199254740992.0); }

void jo_fill_normal(uint64_t seed, float* x, size_t n, float mean, float std) {
    uint64_t s = seed;
    for (size_t i = 0; i < n; i += 2) {
        double u1 = unit_open(&s), u2 = unit_open(&s);
        double r = sqrt(-2.0 * log(u1)), t = 6.283185307179586 * u2;
        x[i] = (float)(mean + std * r * cos(t));
        if (i + 1 < n) x[i + 1] = (float)(mean + std * r * sin(t));
    }
}

void jo_fill_outliers(uint64_t seed, float* x, size_t n, float p, float mag) {
    jo_fill_normal(seed, x, n, 0.0f, 1.0f);
    uint64_t s = seed ^ 0xA5A5A5A5DEADBEEFull;
    for (size_t i = 0; i < n; i++) {
        double u = unit_open(&s);
        if (u < p) x[i] = (splitmix64(&s) & 1) ? mag : -mag;
    }
}
