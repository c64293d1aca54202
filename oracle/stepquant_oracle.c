/*
 * STEPQuant CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C, the reference algorithm of STEPQuant's
 * packed-state recurrent update so that the HIP product can be checked
 * against it.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product (stepquant_amd) never calls it.
 *
 * What each function follows (paths relative to the reference repository):
 *   sqo_layout         stepquant/kernels/pool.py:19-66 (packed_layout)
 *   sqo_fit_state      stepquant/quantization.py:49-98 (_fp16_scale, fit_state)
 *   sqo_encode_page    fit_state + page stores of kernels/fused.py:251-282
 *                      (rows_kernel) and :62-127 (column_kernel) with
 *                      kernels/bitpack.py:6-30 (store_words)
 *   sqo_decode_page    kernels/fused.py:18-59 (_read / codec_kernel)
 *   sqo_prepare        kernels/fused.py:155-179 (prepare_inputs_kernel)
 *   sqo_delta_step     stepquant/core.py:5-15 (delta_step)
 *
 * Float32 reductions reproduce PyTorch's CPU summation order, because
 * fit_state's bit-exact output depends on it (quantization.py:106 mean over
 * the value axis, :131-132 sums over the key axis).  The order is that of
 * aten/src/ATen/native/cpu/SumKernel.cpp (cascade_sum): 8-wide float vectors,
 * 4 interleaved accumulators, 16-element cascade levels.  It is pinned by
 * tests/test_oracle_math.py (test_inner_sum_tree_matches_torch,
 * test_outer_sum_tree_matches_torch, test_tree_differs_from_naive_order)
 * against torch itself and by the golden vectors.
 *
 * Compile with -ffp-contract=off: every multiply and add rounds separately,
 * as the reference's PyTorch elementwise ops do.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ fp16 */

/* float -> IEEE half, round to nearest even (torch.Tensor.half()). */
uint16_t sqo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf or nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    }
    if (ax >= 0x477ff000u) { /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax < 0x38800000u) { /* below 2^-14: half subnormal or zero */
        if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to 0 */
        /* value = m * 2^(e-150); half subnormal unit = 2^-24 */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e; /* 2^(e-150)/2^-24 = 2^(e-126) */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    /* normal range */
    uint32_t e = (ax >> 23) - 112u; /* rebias 127 -> 15 */
    uint32_t m = ax & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

float sqo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else { /* subnormal: normalise */
            int s = 0;
            while (!(m & 0x400u)) { m <<= 1; s++; }
            m &= 0x3ffu;
            x = sign | ((uint32_t)(113 - s) << 23) | (m << 13);
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* quantization.py:49-51 _fp16_scale: clamp(2^-24, 65504).half().float() */
static float fp16_scale(float x, uint16_t *bits_out) {
    const float lo = 5.9604644775390625e-08f, hi = 65504.0f;
    float c = x < lo ? lo : x; /* torch.clamp: max(min) order; NaN aside */
    c = c > hi ? hi : c;
    uint16_t h = sqo_f32_to_f16(c);
    if (bits_out) *bits_out = h;
    return sqo_f16_to_f32(h);
}

/* ---------------------------------------------- PyTorch CPU sum ordering */

static int ceil_log2(int64_t x) {
    if (x <= 2) return 1;
    uint64_t v = (uint64_t)x - 1;
    int r = 0;
    while (v) { r++; v >>= 1; }
    return r;
}

/*
 * multi_row_sum of SumKernel.cpp for nrows accumulators: element (i, k) is
 * at in[i*row_stride + k*col_stride]; returns the nrows partial sums.
 */
static void multi_row_sum(const float *in, int64_t row_stride, int64_t col_stride,
                          int64_t size, int nrows, float *out) {
    enum { LEVELS = 4, MAXROWS = 4 };
    int level_power = ceil_log2(size) / 4;
    if (level_power < 4) level_power = 4;
    const int64_t level_step = (int64_t)1 << level_power;
    const int64_t level_mask = level_step - 1;
    float acc[LEVELS][MAXROWS];
    for (int a = 0; a < LEVELS; a++)
        for (int k = 0; k < MAXROWS; k++) acc[a][k] = 0.0f;
    int64_t i = 0;
    for (; i + level_step <= size;) {
        for (int64_t j = 0; j < level_step; ++j, ++i) {
            const float *b = in + i * row_stride;
            for (int k = 0; k < nrows; k++) acc[0][k] += b[k * col_stride];
        }
        for (int j = 1; j < LEVELS; ++j) {
            for (int k = 0; k < nrows; k++) {
                acc[j][k] += acc[j - 1][k];
                acc[j - 1][k] = 0.0f;
            }
            const int64_t mask = level_mask << (j * level_power);
            if ((i & mask) != 0) break;
        }
    }
    for (; i < size; ++i) {
        const float *b = in + i * row_stride;
        for (int k = 0; k < nrows; k++) acc[0][k] += b[k * col_stride];
    }
    for (int j = 1; j < LEVELS; ++j)
        for (int k = 0; k < nrows; k++) acc[0][k] += acc[j][k];
    for (int k = 0; k < nrows; k++) out[k] = acc[0][k];
}

/* row_sum with four interleaved accumulators (ilp_factor = 4). */
static float row_sum_ilp4(const float *in, int64_t stride, int64_t size) {
    float p[4];
    const int64_t size_ilp = size / 4;
    multi_row_sum(in, stride * 4, stride, size_ilp, 4, p);
    for (int64_t i = size_ilp * 4; i < size; ++i) p[0] += in[i * stride];
    for (int k = 1; k < 4; k++) p[0] += p[k];
    return p[0];
}

/* Sum of n contiguous floats in torch's inner-reduction order. */
float sqo_torch_inner_sum(const float *x, int64_t n) {
    const int L = 8; /* Vectorized<float> width used by the float sum kernel */
    if (n < L) return row_sum_ilp4(x, 1, n);
    const int64_t nvec = n / L;
    float lane[8];
    for (int l = 0; l < L; l++) lane[l] = row_sum_ilp4(x + l, L, nvec);
    float total = 0.0f;
    for (int64_t k = nvec * L; k < n; ++k) total += x[k];
    for (int l = 0; l < L; l++) total += lane[l];
    return total;
}

/*
 * Sum over n rows (stride apart) of one column, in torch's outer-reduction
 * order for a tensor whose contiguous inner dimension has ncols columns:
 * column chunks of 32 use the cascade directly, narrower tails use row_sum.
 */
float sqo_torch_outer_sum(const float *x, int64_t n, int64_t stride, int64_t ncols, int64_t col) {
    if (col < (ncols / 32) * 32) {
        float out;
        multi_row_sum(x, stride, 1, n, 1, &out);
        return out;
    }
    return row_sum_ilp4(x, stride, n);
}

/* ----------------------------------------------------------------- layout */

/*
 * kernels/pool.py:19-66.  offsets: H*K row offsets then H strides (byte
 * storage: H code bases).  rows: H*K (-1 for pivots).  columns: H (-1 for
 * all-pivot heads).  Returns the page size in bytes.
 */
int64_t sqo_layout(const int32_t *bits, int H, int K, int V, int kda, int byte_storage,
                   int group, int32_t *offsets, int32_t *rows, int32_t *columns) {
    int64_t cursor = 0;
    int tile = kda ? 4 : 16;
    if (tile > V) tile = V;
    int32_t *strides = offsets + (int64_t)H * K;
    if (byte_storage) {
        for (int h = 0; h < H; h++) {
            const int32_t *hb = bits + (int64_t)h * K;
            int64_t code_base = cursor;
            int any_int = 0, pivots = 0;
            for (int i = 0; i < K; i++) { any_int |= hb[i] != 16; pivots += hb[i] == 16; }
            if (any_int) cursor += (int64_t)K * V;
            int64_t pivot_base = cursor;
            int pivot_index = 0;
            for (int i = 0; i < K; i++) {
                if (hb[i] == 16) {
                    offsets[(int64_t)h * K + i] = (int32_t)(pivot_base + 2 * (int64_t)pivot_index * V);
                    pivot_index++;
                } else {
                    offsets[(int64_t)h * K + i] = (int32_t)(code_base + i);
                }
            }
            cursor += 2 * (int64_t)pivots * V;
            strides[h] = (int32_t)code_base;
        }
    } else {
        for (int h = 0; h < H; h++) {
            const int32_t *hb = bits + (int64_t)h * K;
            int64_t local = 0;
            for (int i = 0; i < K; i++) {
                if (hb[i] == 16) local = (local + 1) / 2 * 2;
                offsets[(int64_t)h * K + i] = (int32_t)(cursor + local);
                local += (int64_t)tile * hb[i] / 8;
            }
            int64_t stride = (local + 1) / 2 * 2;
            strides[h] = (int32_t)stride;
            cursor += stride * (V / tile);
        }
    }
    cursor = (cursor + 1) / 2 * 2;
    for (int h = 0; h < H; h++) {
        for (int i = 0; i < K; i++) {
            int b = bits[(int64_t)h * K + i];
            rows[(int64_t)h * K + i] = b != 16 ? (int32_t)cursor : -1;
            if (b != 16) cursor += 2 * ((b == 2 && !kda) ? V / group : 1);
        }
    }
    for (int h = 0; h < H; h++) {
        int any_int = 0;
        for (int i = 0; i < K; i++) any_int |= bits[(int64_t)h * K + i] != 16;
        columns[h] = any_int ? (int32_t)cursor : -1;
        if (any_int) cursor += 2 * (int64_t)V;
    }
    if (byte_storage) cursor = (cursor + 15) / 16 * 16;
    return cursor;
}

/* -------------------------------------------------------------- fit_state */

static inline float round_half_even(float y) { return rintf(y); }

/*
 * quantization.py:54-98 fit_state on a dense state x [B,H,K,V].
 * Outputs: z int16 [B,H,K,V]; r fp16 [B,H,K]; c fp16 [B,H,V];
 * r2 fp16 [B,H,K,V/group] (GDN 2-bit heads only, others left untouched);
 * recon f32 [B,H,K,V] (may be NULL).  Returns 0, or -1 on bad arguments.
 */
int sqo_fit_state(const float *x, int B, int H, int K, int V, const int32_t *bits,
                  const float *impact, int kda, int group, int16_t *z_out, uint16_t *r_out,
                  uint16_t *c_out, uint16_t *r2_out, float *recon) {
    const int64_t KV = (int64_t)K * V;
    int any_two = 0;
    if (!kda)
        for (int h = 0; h < H; h++) any_two |= bits[(int64_t)h * K] == 2;
    if (any_two && (group < 1 || V % group)) return -1;
    const int NG = any_two ? V / group : 1;
    float *absx = (float *)malloc(sizeof(float) * (size_t)V);
    float *rfull = (float *)malloc(sizeof(float) * (size_t)KV);
    float *scaled = (float *)malloc(sizeof(float) * (size_t)KV);
    float *tmpn = (float *)malloc(sizeof(float) * (size_t)KV);
    float *tmpd = (float *)malloc(sizeof(float) * (size_t)KV);
    float *qmax = (float *)malloc(sizeof(float) * (size_t)K);
    float *norm = (float *)malloc(sizeof(float) * (size_t)K);
    float *c0 = (float *)malloc(sizeof(float) * (size_t)V);
    float *c1 = (float *)malloc(sizeof(float) * (size_t)V);
    float *zf = (float *)malloc(sizeof(float) * (size_t)KV);
    if (!absx || !rfull || !scaled || !tmpn || !tmpd || !qmax || !norm || !c0 || !c1 || !zf) return -2;
    for (int b = 0; b < B; b++) {
        for (int h = 0; h < H; h++) {
            const float *xs = x + ((int64_t)b * H + h) * KV;
            const int32_t *hb = bits + (int64_t)h * K;
            const float *hw = impact + (int64_t)h * K;
            const int two = !kda && hb[0] == 2;
            for (int i = 0; i < K; i++) {
                int bc = hb[i] < 8 ? hb[i] : 8;
                qmax[i] = ldexpf(1.0f, bc - 1) - 1.0f;
                norm[i] = kda ? ldexpf(1.0f, 8 - bc) : 1.0f;
                if (two) qmax[i] = 3.0f;
                for (int j = 0; j < V; j++) absx[j] = fabsf(xs[(int64_t)i * V + j]);
                float mean = sqo_torch_inner_sum(absx, V) / (float)V;
                float m = mean < 1e-20f ? 1e-20f : mean;
                uint16_t rb;
                float r = fp16_scale(sqrtf(m / hw[i]), &rb);
                r_out[((int64_t)b * H + h) * K + i] = rb;
                for (int j = 0; j < V; j++) rfull[(int64_t)i * V + j] = r;
                if (two) {
                    for (int g = 0; g < NG; g++) {
                        float gm = sqo_torch_inner_sum(absx + (int64_t)g * group, group) / (float)group;
                        float mm = gm < 1e-20f ? 1e-20f : gm;
                        uint16_t gb;
                        float r2 = fp16_scale(sqrtf(mm / hw[i]), &gb);
                        r2_out[(((int64_t)b * H + h) * K + i) * NG + g] = gb;
                        for (int j = g * group; j < (g + 1) * group; j++) rfull[(int64_t)i * V + j] = r2;
                    }
                }
            }
            for (int64_t e = 0; e < KV; e++) scaled[e] = xs[e] / rfull[e];
            /* c0 = amax over key rows of where(integer, |scaled| / (qmax*norm), 0) */
            for (int j = 0; j < V; j++) {
                float mx = 0.0f;
                for (int i = 0; i < K; i++) {
                    float t = hb[i] != 16 ? fabsf(scaled[(int64_t)i * V + j]) / (qmax[i] * norm[i]) : 0.0f;
                    if (t > mx) mx = t;
                }
                c0[j] = fp16_scale(mx, NULL);
            }
            /* encode(c0), weighted refit */
            for (int i = 0; i < K; i++) {
                float wsq = (hw[i] * hw[i]) * (hb[i] != 16 ? 1.0f : 0.0f);
                for (int j = 0; j < V; j++) {
                    int64_t e = (int64_t)i * V + j;
                    float y = (scaled[e] / c0[j]) / norm[i];
                    float z;
                    if (two) z = (y >= 0.0f ? 1.0f : -1.0f) * (fabsf(y) >= 2.0f ? 3.0f : 1.0f);
                    else {
                        z = round_half_even(y);
                        z = z > -qmax[i] ? z : -qmax[i];
                        z = z < qmax[i] ? z : qmax[i];
                    }
                    float v = (rfull[e] * norm[i]) * z;
                    tmpn[e] = (wsq * v) * xs[e];
                    tmpd[e] = wsq * (v * v);
                }
            }
            for (int j = 0; j < V; j++) {
                float num = sqo_torch_outer_sum(tmpn + j, K, V, V, j);
                float den = sqo_torch_outer_sum(tmpd + j, K, V, V, j);
                float den_c = den < 1e-30f ? 1e-30f : den;
                float cc = den > 0.0f ? num / den_c : c0[j];
                uint16_t cb;
                c1[j] = fp16_scale(cc, &cb);
                c_out[((int64_t)b * H + h) * V + j] = cb;
            }
            for (int i = 0; i < K; i++) {
                for (int j = 0; j < V; j++) {
                    int64_t e = (int64_t)i * V + j;
                    float y = (scaled[e] / c1[j]) / norm[i];
                    float z;
                    if (two) z = (y >= 0.0f ? 1.0f : -1.0f) * (fabsf(y) >= 2.0f ? 3.0f : 1.0f);
                    else {
                        z = round_half_even(y);
                        z = z > -qmax[i] ? z : -qmax[i];
                        z = z < qmax[i] ? z : qmax[i];
                    }
                    zf[e] = z;
                    z_out[((int64_t)b * H + h) * KV + e] = (int16_t)z;
                    if (recon) {
                        float rec = hb[i] != 16 ? ((rfull[e] * c1[j]) * norm[i]) * z
                                                : sqo_f16_to_f32(sqo_f32_to_f16(xs[e]));
                        recon[((int64_t)b * H + h) * KV + e] = rec;
                    }
                }
            }
        }
    }
    free(absx); free(rfull); free(scaled); free(tmpn); free(tmpd);
    free(qmax); free(norm); free(c0); free(c1); free(zf);
    return 0;
}

/* ------------------------------------------------------------ page codec */

static void put_bits(uint8_t *p, int64_t bitpos, uint32_t code, int width) {
    for (int t = 0; t < width; t++) {
        int64_t bp = bitpos + t;
        uint8_t m = (uint8_t)(1u << (bp & 7));
        if ((code >> t) & 1u) p[bp >> 3] |= m; else p[bp >> 3] &= (uint8_t)~m;
    }
}

static uint32_t get_bits(const uint8_t *p, int64_t bitpos, int width) {
    uint32_t v = 0;
    for (int t = 0; t < width; t++) {
        int64_t bp = bitpos + t;
        v |= (uint32_t)((p[bp >> 3] >> (bp & 7)) & 1u) << t;
    }
    return v;
}

static void put_half(uint8_t *p, int64_t byte, uint16_t h) {
    p[byte] = (uint8_t)(h & 0xff);
    p[byte + 1] = (uint8_t)(h >> 8);
}

static uint16_t get_half(const uint8_t *p, int64_t byte) {
    return (uint16_t)(p[byte] | ((uint16_t)p[byte + 1] << 8));
}

/* Byte address of value j of a packed row, and its bit position (pool.py:19-66). */
static int64_t packed_bit(const int32_t *offsets, int H, int K, int V, int kda, int h, int i,
                          int j, int width) {
    int tile = kda ? 4 : 16;
    if (tile > V) tile = V;
    int64_t off = offsets[(int64_t)h * K + i];
    int64_t stride = offsets[(int64_t)H * K + h];
    return (off + (int64_t)(j / tile) * stride) * 8 + (int64_t)(j % tile) * width;
}

/*
 * Write fit_state(x) into page slots (packed storage; byte storage follows
 * kernels/fit.py:295-299 int8 carriers).  slot <= 0 entries are skipped.
 */
int sqo_encode_page(const float *x, int B, int H, int K, int V, const int32_t *bits,
                    const float *impact, int kda, int group, int byte_storage,
                    const int32_t *offsets, const int32_t *rows, const int32_t *columns,
                    const int64_t *slots, uint8_t *data, int64_t page_bytes) {
    const int64_t KV = (int64_t)K * V;
    int16_t *z = (int16_t *)malloc(sizeof(int16_t) * (size_t)(B * KV * H));
    uint16_t *r = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(B * H * K));
    uint16_t *c = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(B * H * V));
    int NG = (!kda && group > 0 && V % group == 0) ? V / group : 1;
    uint16_t *r2 = (uint16_t *)calloc((size_t)(B * H * K * NG), sizeof(uint16_t));
    if (!z || !r || !c || !r2) return -2;
    int rc = sqo_fit_state(x, B, H, K, V, bits, impact, kda, group, z, r, c, r2, NULL);
    if (rc) return rc;
    for (int b = 0; b < B; b++) {
        if (slots[b] <= 0) continue;
        uint8_t *page = data + slots[b] * page_bytes;
        for (int h = 0; h < H; h++) {
            const int32_t *hb = bits + (int64_t)h * K;
            const int two = !kda && hb[0] == 2;
            const float *xs = x + ((int64_t)b * H + h) * KV;
            for (int i = 0; i < K; i++) {
                int bi = hb[i];
                if (bi == 16) {
                    for (int j = 0; j < V; j++) {
                        int64_t byte;
                        if (byte_storage) byte = offsets[(int64_t)h * K + i] + 2 * (int64_t)j;
                        else byte = packed_bit(offsets, H, K, V, kda, h, i, j, 16) / 8;
                        put_half(page, byte, sqo_f32_to_f16(xs[(int64_t)i * V + j]));
                    }
                    continue;
                }
                int64_t ro = rows[(int64_t)h * K + i];
                if (two) {
                    for (int g = 0; g < NG; g++)
                        put_half(page, ro + 2 * g, r2[(((int64_t)b * H + h) * K + i) * NG + g]);
                } else {
                    put_half(page, ro, r[((int64_t)b * H + h) * K + i]);
                }
                int qm = (1 << ((bi < 8 ? bi : 8) - 1)) - 1;
                for (int j = 0; j < V; j++) {
                    int zz = z[((int64_t)b * H + h) * KV + (int64_t)i * V + j];
                    if (byte_storage) {
                        int64_t base = offsets[(int64_t)H * K + h];
                        int carrier = kda ? zz * (1 << (8 - bi)) : zz;
                        page[base + i + (int64_t)j * K] = (uint8_t)(int8_t)carrier;
                    } else {
                        uint32_t code = two ? (uint32_t)((zz + 3) / 2) : (uint32_t)(zz + qm);
                        put_bits(page, packed_bit(offsets, H, K, V, kda, h, i, j, bi), code, bi);
                    }
                }
            }
            if (columns[h] >= 0)
                for (int j = 0; j < V; j++)
                    put_half(page, columns[h] + 2 * (int64_t)j, c[((int64_t)b * H + h) * V + j]);
        }
    }
    free(z); free(r); free(c); free(r2);
    return 0;
}

/* Page -> dense fp32 state (kernels/fused.py:18-59; byte_codec.py:6-28).  slot <= 0 -> zeros. */
int sqo_decode_page(const uint8_t *data, int64_t page_bytes, const int64_t *slots, int B, int H,
                    int K, int V, const int32_t *bits, int kda, int group, int byte_storage,
                    const int32_t *offsets, const int32_t *rows, const int32_t *columns,
                    float *state) {
    const int64_t KV = (int64_t)K * V;
    for (int b = 0; b < B; b++) {
        float *out = state + (int64_t)b * H * KV;
        if (slots[b] <= 0) {
            memset(out, 0, sizeof(float) * (size_t)(H * KV));
            continue;
        }
        const uint8_t *page = data + slots[b] * page_bytes;
        for (int h = 0; h < H; h++) {
            const int32_t *hb = bits + (int64_t)h * K;
            for (int i = 0; i < K; i++) {
                int bi = hb[i];
                for (int j = 0; j < V; j++) {
                    float val;
                    if (bi == 16) {
                        int64_t byte = byte_storage ? offsets[(int64_t)h * K + i] + 2 * (int64_t)j
                                                    : packed_bit(offsets, H, K, V, kda, h, i, j, 16) / 8;
                        val = sqo_f16_to_f32(get_half(page, byte));
                    } else {
                        int bc = bi < 8 ? bi : 8;
                        float z;
                        if (byte_storage) {
                            int64_t base = offsets[(int64_t)H * K + h];
                            z = (float)(int8_t)page[base + i + (int64_t)j * K];
                        } else {
                            uint32_t code = get_bits(page, packed_bit(offsets, H, K, V, kda, h, i, j, bi), bi);
                            if (kda) z = (float)((int)code - ((1 << (bc - 1)) - 1)) * ldexpf(1.0f, 8 - bc);
                            else if (bi == 2) z = 2.0f * (float)code - 3.0f;
                            else z = (float)((int)code - ((1 << (bc - 1)) - 1));
                        }
                        int gi = (!kda && bi == 2) ? j / group : 0;
                        float r = sqo_f16_to_f32(get_half(page, rows[(int64_t)h * K + i] + 2 * (int64_t)gi));
                        float c = columns[h] >= 0 ? sqo_f16_to_f32(get_half(page, columns[h] + 2 * (int64_t)j)) : 0.0f;
                        val = (r * c) * z;
                    }
                    out[(int64_t)h * KV + (int64_t)i * V + j] = val;
                }
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------- decode-step math */

/*
 * Input preparation (kernels/fused.py:155-179): optional L2 normalisation
 * with eps 1e-6, query scale, raw gates g = -exp(A_log)*softplus_20(a+bias),
 * beta = sigmoid(b).  q,k are read per key head (GQA: value head h uses key
 * head h / (H/HK)); outputs qp,kp [B,H,K], logdecay [B,H] or [B,H,K],
 * beta_out [B,H].
 */
void sqo_prepare(const float *q, const float *k, int64_t qs, int64_t ks, const float *g,
                 const float *beta, const float *a_log, const float *dt_bias, int B, int H,
                 int HK, int K, int kda, int normalize, float scale, float *qp, float *kp,
                 float *logdecay, float *beta_out) {
    for (int b = 0; b < B; b++) {
        for (int h = 0; h < H; h++) {
            int hk = h / (H / HK);
            const float *qr = q + (int64_t)b * qs + (int64_t)hk * K;
            const float *kr = k + (int64_t)b * ks + (int64_t)hk * K;
            float sq = 0.0f, sk = 0.0f;
            for (int i = 0; i < K; i++) { sq += qr[i] * qr[i]; sk += kr[i] * kr[i]; }
            float nq = normalize ? 1.0f / sqrtf(sq + 1e-6f) : 1.0f;
            float nk = normalize ? 1.0f / sqrtf(sk + 1e-6f) : 1.0f;
            for (int i = 0; i < K; i++) {
                qp[((int64_t)b * H + h) * K + i] = (qr[i] * nq) * scale;
                kp[((int64_t)b * H + h) * K + i] = kr[i] * nk;
            }
            float bt = beta[(int64_t)b * H + h];
            if (a_log) bt = 1.0f / (1.0f + expf(-bt));
            beta_out[(int64_t)b * H + h] = bt;
            int n = kda ? K : 1;
            for (int i = 0; i < n; i++) {
                int64_t gi = kda ? ((int64_t)b * H + h) * K + i : (int64_t)b * H + h;
                float gv = g[gi];
                if (a_log) {
                    float u = gv + dt_bias[kda ? (int64_t)h * K + i : h];
                    float sp = u > 20.0f ? u : logf(1.0f + expf(u < 20.0f ? u : 20.0f));
                    gv = -expf(a_log[h]) * sp;
                }
                logdecay[gi] = gv;
            }
        }
    }
}

/*
 * core.py:5-15 delta_step on prepared inputs: retained = S*exp(g);
 * residual = v - k^T retained; S' = retained + k (beta residual)^T;
 * o = q^T S'.  state/updated [B,H,K,V], v/out [B,H,V].
 */
void sqo_delta_step(const float *state, const float *q, const float *k, const float *v,
                    const float *logdecay, const float *beta, int B, int H, int K, int V, int kda,
                    float *out, float *updated) {
    const int64_t KV = (int64_t)K * V;
    for (int b = 0; b < B; b++) {
        for (int h = 0; h < H; h++) {
            int64_t bh = (int64_t)b * H + h;
            const float *S = state + bh * KV;
            float *U = updated + bh * KV;
            const float *qr = q + bh * K, *kr = k + bh * K, *vr = v + bh * V;
            for (int i = 0; i < K; i++) {
                float d = expf(kda ? logdecay[bh * K + i] : logdecay[bh]);
                for (int j = 0; j < V; j++) U[(int64_t)i * V + j] = S[(int64_t)i * V + j] * d;
            }
            for (int j = 0; j < V; j++) {
                float s = 0.0f;
                for (int i = 0; i < K; i++) s += kr[i] * U[(int64_t)i * V + j];
                float delta = beta[bh] * (vr[j] - s);
                float o = 0.0f;
                for (int i = 0; i < K; i++) {
                    float x = U[(int64_t)i * V + j] + kr[i] * delta;
                    U[(int64_t)i * V + j] = x;
                    o += qr[i] * x;
                }
                out[bh * V + j] = o;
            }
        }
    }
}
